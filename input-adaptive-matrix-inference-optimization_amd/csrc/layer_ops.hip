// Layer kernels around the sparse GEMV: RMSNorm + gain, residual add,
// SiLU-gated activation, RoPE + KV append, decode attention, embedding
// gather and greedy argmax (aux.cl, matrix.cl:27-32, bucketMul.cl:517-520).
#include <hip/hip_fp16.h>

#include <cmath>

#include "accum.h"
#include "internal.h"
#include "layer_ops.h"
#include "wave.h"

namespace iam {

__device__ __forceinline__ float h2f(uint16_t b) { return __half2float(__ushort_as_half(b)); }

// ------------------------------------------------------------- RMSNorm ---
// rmsNorm32fast (aux.cl:156-196): 256 threads, n/256 consecutive squares per
// thread summed in order, a 256-way tree, scale = 1/sqrt(sum/n + eps)
// (rounded from double); then the fp16 gain (mul16x32, aux.cl:434-440).
// With `delta` the residual add32 (bucketMul.cl:517-520) is applied to h
// first and written back.  Each thread's values, deltas and gains are loaded
// with 16-byte loads issued together (n/256 must be a multiple of 4 and at
// most kNormMaxPer) and kept in registers for the second pass.
constexpr int kNormMaxPer = 64;

template <int PER>
__global__ __launch_bounds__(256) void k_rmsnorm(float* __restrict__ h, const float* __restrict__ delta,
                                                 const uint16_t* __restrict__ gain, float eps,
                                                 float* __restrict__ out)
{
#pragma clang fp contract(off)
    __shared__ float part[256];
    const int tid = threadIdx.x;
    constexpr int n = PER * 256;
    const int b0 = tid * PER;
    float v[PER];
    uint2 g4[PER / 4];
#pragma unroll
    for (int k = 0; k < PER / 4; k++) {
        const float4 a = *reinterpret_cast<const float4*>(h + b0 + 4 * k);
        v[4 * k] = a.x;
        v[4 * k + 1] = a.y;
        v[4 * k + 2] = a.z;
        v[4 * k + 3] = a.w;
        g4[k] = *reinterpret_cast<const uint2*>(gain + b0 + 4 * k);
    }
    if (delta) {
        float dv[PER];
#pragma unroll
        for (int k = 0; k < PER / 4; k++) {
            const float4 a = *reinterpret_cast<const float4*>(delta + b0 + 4 * k);
            dv[4 * k] = a.x;
            dv[4 * k + 1] = a.y;
            dv[4 * k + 2] = a.z;
            dv[4 * k + 3] = a.w;
        }
#pragma unroll
        for (int k = 0; k < PER; k++) v[k] = __fadd_rn(v[k], dv[k]);
#pragma unroll
        for (int k = 0; k < PER / 4; k++)
            *reinterpret_cast<float4*>(h + b0 + 4 * k) = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
    }
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; k++) s = __fadd_rn(s, __fmul_rn(v[k], v[k]));
    part[tid] = s;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if (tid < st) part[tid] = __fadd_rn(part[tid], part[tid + st]);
        __syncthreads();
    }
    const float mean = __fdiv_rn(part[0], (float)n);
    const float scale = (float)(1.0 / sqrt((double)__fadd_rn(mean, eps)));
#pragma unroll
    for (int k = 0; k < PER / 4; k++) {
        float o[4];
        const uint32_t gw[2] = {g4[k].x, g4[k].y};
#pragma unroll
        for (int e = 0; e < 4; e++)
            o[e] = __fmul_rn(h2f((uint16_t)(gw[e >> 1] >> ((e & 1) * 16))), __fmul_rn(v[4 * k + e], scale));
        *reinterpret_cast<float4*>(out + b0 + 4 * k) = make_float4(o[0], o[1], o[2], o[3]);
    }
}

// h_out = h + (float)delta (add32 of an accumulated delta, bucketMul.cl:517-520),
// then RMSNorm + gain of h_out into out, for any n = 256 * PER (PER <= 64):
// the same order of sums as k_rmsnorm, two passes over memory.  Used by
// models wider than the 4096 inputs the walk normalises itself.
template <typename Dt>
__global__ __launch_bounds__(256) void k_resnorm(const float* __restrict__ h, const Dt* __restrict__ delta,
                                                 float* __restrict__ h_out, const uint16_t* __restrict__ gain,
                                                 float eps, int n, float* __restrict__ out)
{
#pragma clang fp contract(off)
    __shared__ float part[256];
    const int tid = threadIdx.x;
    const int per = n / 256;
    const int b0 = tid * per;
    float s = 0.0f;
    for (int k = 0; k < per; k++) {
        float v = h[b0 + k];
        if (delta) v = __fadd_rn(v, (float)delta[b0 + k]);
        if (h_out) h_out[b0 + k] = v;
        s = __fadd_rn(s, __fmul_rn(v, v));
    }
    part[tid] = s;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
        if (tid < st) part[tid] = __fadd_rn(part[tid], part[tid + st]);
        __syncthreads();
    }
    const float mean = __fdiv_rn(part[0], (float)n);
    const float scale = (float)(1.0 / sqrt((double)__fadd_rn(mean, eps)));
    for (int k = 0; k < per; k++) {
        float v = h[b0 + k];
        if (delta) v = __fadd_rn(v, (float)delta[b0 + k]);
        out[b0 + k] = __fmul_rn(h2f(gain[b0 + k]), __fmul_rn(v, scale));
    }
}

// ------------------------------------------------------------ residual ---
__global__ void k_add(const float* __restrict__ a, const float* __restrict__ b, int n,
                      float* __restrict__ out)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = __fadd_rn(a[i], b[i]);
}

// ---------------------------------------------------------------- SiLU ---
// silu32 (matrix.cl:27-32): out = x3 * x1 / (1 + exp(-x1)), x1 = gate,
// x3 = up, evaluated in fp64 and rounded once (the value the fp32 kernel
// approximates)
__global__ void k_silu_mul(const float* __restrict__ g, const float* __restrict__ u, int n,
                           float* __restrict__ out)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const double x1 = (double)g[i];
        out[i] = (float)((double)u[i] * x1 / (1.0 + exp(-x1)));
    }
}

// ---------------------------------------------------------------- RoPE ---

__global__ void k_rope(const float* __restrict__ in, const float* __restrict__ table,
                       const int* __restrict__ pos_p, int n_heads, int hd, int max_pos,
                       float* __restrict__ out)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int pos = *pos_p;
    if (i >= n_heads * hd || pos < 0 || pos >= max_pos) return;
    const int h = i / hd, d = i - h * hd;
    out[i] = rope_one(in + h * hd, table + (size_t)pos * hd, d, hd / 2);
}

// RoPE of q and k, then store k (after RoPE) and v at the position as fp16
// (attention.hpp:172-189 with the copies of :281-309; the reference applies
// RoPE to the GQA-repeated k, which has the same values per repeated head).
__global__ void k_rope_kv(const float* __restrict__ q, const float* __restrict__ k,
                          const float* __restrict__ v, const float* __restrict__ table,
                          const int* __restrict__ pos_p, int n_heads, int n_kv, int hd, int max_ctx,
                          float* __restrict__ q_out, uint16_t* __restrict__ kc,
                          uint16_t* __restrict__ vc)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int pos = *pos_p;
    if (pos < 0 || pos >= max_ctx) return;
    const int nq = n_heads * hd, nk = n_kv * hd;
    const float* row = table + (size_t)pos * hd;
    const int half = hd / 2;
    if (i < nq) {
        const int h = i / hd, d = i - h * hd;
        q_out[i] = rope_one(q + h * hd, row, d, half);
    } else if (i < nq + nk) {
        const int j = i - nq;
        const int h = j / hd, d = j - h * hd;
        kc[(size_t)pos * nk + j] = __half_as_ushort(__float2half_rn(rope_one(k + h * hd, row, d, half)));
    } else if (i < nq + 2 * nk) {
        const int j = i - nq - nk;
        vc[(size_t)pos * nk + j] = __half_as_ushort(__float2half_rn(v[j]));
    }
}

// ------------------------------------------------------------ attention ---
// Decode attention over an fp16 GQA cache, split over the context.  The
// context is cut into chunks of 64 positions, dealt in runs of consecutive
// chunks to at most kAttnGroups workgroups per head group.  Workgroup (head
// group, run) takes HPW query heads of one KV head (2 where a KV head's
// query heads pair up, else 1; repeat4x32, aux.cl:266-275, without
// materialising the repeat); the head groups of one KV head sit in
// workgroups whose index is equal modulo n_kv, so with 8 KV heads they run on
// one XCD and share the K and V rows in its L2.  Each chunk's K and V rows
// are loaded into LDS, 16 bytes per thread (the next chunk's loads in flight
// during this one's arithmetic).  Dot products (dotSetScore2, aux.cl:497-540,
// s = q.k / sqrt(hd)): lane = position, wave w adds dimensions 16w..16w+15
// for every head of the group (each K value converted once) with q
// broadcast from LDS, and the waves' sums are added in wave order; wave j
// takes p = exp(s) of head j (sum_of_exps32_mx / softmax_add32_mx,
// aux.cl:204-225: the reference's softmax has no maximum subtracted, so the
// runs' sums add up directly) and their sum.  p.V: lane l takes dimensions 2l
// and 2l+1 over the 8 positions 8w..8w+7 of each chunk, for every head, and
// the waves' sums are added in wave order.  The runs' sums p*V and sums of p
// then meet in o and l for the consumer (the o projection's walk, which
// divides x = o / l), or, for the standalone call, out = o / l (sumScores32,
// aux.cl:370-384).  In the model, while a head group has at most
// atomic_splits runs (always: at most kAttnGroups), each run adds its sums
// into o and l with fp64 atomics (the sums within an fp64 rounding of the
// exact ones, whatever the order).  Otherwise each run writes its sums to
// its heads' slots of the partials with atomic exchanges, waits for them to
// be performed and arrives at its head group's counter; the last run to
// arrive adds the slots in run order (no two runs add to one address, so the
// sums do not depend on arrival order) and writes o and l, or out.  With the
// projection accumulators as input the workgroup also applies RoPE to q and
// k (rope_mx, aux.cl:227-248, table row of the position), and the run holding
// the position uses the new K and V rows from LDS; the workgroup of the KV
// head's first query heads appends them to the cache (attention.hpp:281-309).
// Acc = double evaluates every product (exact: fp32 x fp16), exponential and
// sum in fp64 (a score above log(DBL_MAX) ~ 709.78 overflows, as the
// reference's fp32 exp does above 88.72); Acc = float in fp32.
constexpr int kAttnChunk = 64;
constexpr int kAttnMaxRep = 8;
constexpr int kMaxAttnSplits = 128;   // max_ctx up to 8192
constexpr int kAttnThreads = 512;     // 8 waves
constexpr int kAttnMaxHeads = 512;    // 64 KV heads x 8
constexpr int kAttnGroups = 32;       // workgroups per head group at most (runs of consecutive chunks)
// workgroups per head group of a launch over a context of up to max_ctx positions
static int attn_runs(int max_ctx) { return std::min((max_ctx + kAttnChunk - 1) / kAttnChunk, kAttnGroups); }
// doubles per run and query head in the partials: o (128), the softmax
// sum, padded to 64 bytes
constexpr int kAttnPartStride = 128 + 8;

template <typename Acc>
__device__ __forceinline__ Acc acc_exp(Acc x);
template <>
__device__ __forceinline__ float acc_exp<float>(float x) { return expf(x); }
template <>
__device__ __forceinline__ double acc_exp<double>(double x) { return exp(x); }

struct AttnArgs {
    const float* q;          // queries after RoPE (fp32), or null: from qkv_acc
    const void* qkv_acc;     // the q | k | v accumulators of the projection walk (fp64)
    const float* rope;       // RoPE table [max_ctx][64][2] (qkv_acc mode)
    uint16_t* kc;            // fp16 K rows [max_ctx][n_kv][128] of the layer
    uint16_t* vc;            // fp16 V rows, same layout
    const int* pos;
    int n_heads, n_kv, max_ctx;
    void* acc;               // o [n_heads][128], then l [n_heads] (fp64) (model mode)
    void* part;              // the runs' partial sums [n_heads][runs][kAttnPartStride] (fp64)
    float* out;              // standalone: out = o / l, stored by the last run of each head group
    uint32_t* head_ctr;      // [n_heads] arrival counters (a head group's first head's), zero on
                             // entry (left zero)
    void* zero_p;            // accumulator words cleared by this launch
    int zero_n;
    int atomic_splits;       // model: runs per head group up to which o and l are added with atomics
    int kv_copies;           // qkv_acc: 2 when k and v have second copies after v (added here)
};

// LDS copies of the split's K and V rows: 128 fp16 + 8 of padding (68
// words).  A 16-byte LDS access is served 16 lanes at a time over 64 banks
// of 4 bytes: the dot products read one K row per lane, and 68-word rows
// put 16 consecutive ones on 16 disjoint groups of 4 banks; p.V reads 4
// bytes per lane of one V row (64 lanes, 64 banks).
constexpr int kAttnRowStride = 128 + 8;

template <typename Acc, int HPW>
__global__ __launch_bounds__(kAttnThreads) void k_attn(AttnArgs a, Acc scale)
{
#pragma clang fp contract(off)
    constexpr int HD = 128, RS = kAttnRowStride, DH = HD / 2, NW = kAttnThreads / 64;
    static_assert(HPW == 1 || HPW == 2, "one or two query heads per workgroup");
    __shared__ __align__(16) uint16_t sk[kAttnChunk * RS];
    __shared__ __align__(16) uint16_t sv[kAttnChunk * RS];
    __shared__ __align__(16) Acc sq[HPW][HD];
    __shared__ Acc ss[HPW][NW][kAttnChunk];     // the waves' dot products
    __shared__ Acc sp[HPW][kAttnChunk];         // p
    __shared__ __align__(16) Acc so[NW][HPW][HD];   // the waves' p.V
    __shared__ double sl[HPW];
    __shared__ int s_last;
    zero_share<double>(a.zero_p, a.zero_n, kAttnThreads);
    const int rep = a.n_heads / a.n_kv;
    const int kvh = blockIdx.x % a.n_kv;
    const int r = blockIdx.x / a.n_kv;      // this workgroup's heads among the KV head's
    const int h0 = kvh * rep + r * HPW;     // its first query head
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int pos = *a.pos;
    const int n_tok = min(pos + 1, a.max_ctx);
    // the context's chunks of 64 positions, dealt to at most kAttnGroups
    // workgroups per head group in runs of G consecutive chunks
    const int nch = (n_tok + kAttnChunk - 1) / kAttnChunk;
    const int G = (nch + kAttnGroups - 1) / kAttnGroups;
    const int ng = (nch + G - 1) / G;       // workgroups of these heads with chunks
    const int grp = blockIdx.y;
    if (grp >= ng) return;                  // past the context: neither written nor counted
    const int c0 = grp * G, c1 = min(nch, c0 + G);
    const bool pos_ok = pos >= 0 && pos < a.max_ctx;
    const double* A = reinterpret_cast<const double*>(a.qkv_acc);
    // waves 0 .. 2*HPW-1: q of head h0 + w/2, dimension (w%2)*64 + lane; with
    // the accumulators, the rotation pair (lane, 64 + lane)
    constexpr int WK = 2 * HPW;             // the waves that form the new k and v
    float c = 1.0f, sn = 0.0f;
    if (A && pos_ok && w < WK + 2) {
        c = a.rope[(size_t)pos * HD + 2 * lane];
        sn = a.rope[(size_t)pos * HD + 2 * lane + 1];
    }
    if (w < 2 * HPW) {
        const int hq = h0 + (w >> 1), hf = w & 1;
        float qv;
        if (A) {
            const float lo = (float)A[(size_t)hq * HD + lane], hi = (float)A[(size_t)hq * HD + DH + lane];
            qv = hf == 0 ? __fsub_rn(__fmul_rn(lo, c), __fmul_rn(hi, sn))    // rope_mx: d < 64
                         : __fadd_rn(__fmul_rn(hi, c), __fmul_rn(lo, sn));   // d >= 64
        } else {
            qv = a.q[(size_t)hq * HD + hf * DH + lane];
        }
        sq[w >> 1][hf * DH + lane] = (Acc)qv;
    }
    // waves WK and WK + 1 of the run holding the new position: its k (after
    // RoPE) and v from the accumulators, rounded to fp16; the workgroup of the
    // KV head's first query head appends them to the cache
    const bool fresh = A && pos_ok && pos >= c0 * kAttnChunk && pos < c1 * kAttnChunk;
    uint16_t fr0 = 0, fr1 = 0;
    if (fresh && w >= WK && w < WK + 2) {
        const bool isk = w == WK;
        const int nq = a.n_heads * HD, nk = a.n_kv * HD;
        const size_t base = (size_t)(isk ? nq : nq + nk) + (size_t)kvh * HD;
        const size_t base2 = a.kv_copies > 1 ? base + 2 * (size_t)nk : base;   // the odd slices' copy
        // all four loads unconditional (a single copy re-reads its own
        // values), so they go out together and share one wait
        const double x0 = A[base + lane], x1 = A[base + DH + lane];
        const double y0 = A[base2 + lane], y1 = A[base2 + DH + lane];
        const float lo = (float)(a.kv_copies > 1 ? x0 + y0 : x0);
        const float hi = (float)(a.kv_copies > 1 ? x1 + y1 : x1);
        float o0 = lo, o1 = hi;
        if (isk) {
            o0 = __fsub_rn(__fmul_rn(lo, c), __fmul_rn(hi, sn));
            o1 = __fadd_rn(__fmul_rn(hi, c), __fmul_rn(lo, sn));
        }
        fr0 = __half_as_ushort(__float2half_rn(o0));
        fr1 = __half_as_ushort(__float2half_rn(o1));
        if (r == 0) {
            uint16_t* crow = (isk ? a.kc : a.vc) + ((size_t)pos * a.n_kv + kvh) * HD;
            crow[lane] = fr0;
            crow[DH + lane] = fr1;
        }
    }
    // K and V pieces (16 bytes) of chunk ch: thread tid takes pieces tid and
    // tid + 512 (row = piece / 16); pieces past the chunk re-read its last one
    static_assert(kAttnChunk * (HD / 8) == 2 * kAttnThreads, "two pieces per thread");
    uint4 ka, kb, va, vb;
    auto load_chunk = [&](int ch) __attribute__((always_inline)) {
        const int t0 = ch * kAttnChunk, nt = min(kAttnChunk, n_tok - t0), pieces = nt * (HD / 8);
        const int i0 = min(tid, pieces - 1), i1 = min(kAttnThreads + tid, pieces - 1);
        const size_t g0 = ((size_t)(t0 + (i0 >> 4)) * a.n_kv + kvh) * HD + (i0 & 15) * 8;
        const size_t g1 = ((size_t)(t0 + (i1 >> 4)) * a.n_kv + kvh) * HD + (i1 & 15) * 8;
        ka = *reinterpret_cast<const uint4*>(a.kc + g0);
        kb = *reinterpret_cast<const uint4*>(a.kc + g1);
        va = *reinterpret_cast<const uint4*>(a.vc + g0);
        vb = *reinterpret_cast<const uint4*>(a.vc + g1);
    };
    load_chunk(c0);
    Acc o[HPW][2];   // p.V of dimensions 2*lane, 2*lane + 1 over this wave's positions, per head
#pragma unroll
    for (int j = 0; j < HPW; j++) o[j][0] = o[j][1] = (Acc)0;
    Acc l = (Acc)0;   // wave j < HPW: the sum of p of head h0 + j
    for (int ch = c0; ch < c1; ch++) {
        const int t0 = ch * kAttnChunk, nt = min(kAttnChunk, n_tok - t0), pieces = nt * (HD / 8);
        // the chunk's rows into LDS (the new row from the accumulators), then
        // the next chunk's loads go out
        {
            const int i0 = tid, i1 = kAttnThreads + tid;
            if (i0 < pieces && !(fresh && t0 + (i0 >> 4) == pos)) {
                const int oo = (i0 >> 4) * RS + (i0 & 15) * 8;
                *reinterpret_cast<uint4*>(sk + oo) = ka;
                *reinterpret_cast<uint4*>(sv + oo) = va;
            }
            if (i1 < pieces && !(fresh && t0 + (i1 >> 4) == pos)) {
                const int oo = (i1 >> 4) * RS + (i1 & 15) * 8;
                *reinterpret_cast<uint4*>(sk + oo) = kb;
                *reinterpret_cast<uint4*>(sv + oo) = vb;
            }
        }
        if (fresh && w >= WK && w < WK + 2 && pos >= t0 && pos < t0 + kAttnChunk) {
            uint16_t* lrow = (w == WK ? sk : sv) + (pos - t0) * RS;
            lrow[lane] = fr0;
            lrow[DH + lane] = fr1;
        }
        if (ch + 1 < c1) load_chunk(ch + 1);
        __syncthreads();
        // dot products: position t0 + lane over dimensions 16w..16w+15, each
        // K value converted once for the HPW heads (two chains per head, then
        // added), then the waves' sums in wave order
        {
            Acc s0[HPW], s1[HPW];
#pragma unroll
            for (int j = 0; j < HPW; j++) s0[j] = s1[j] = (Acc)0;
            const uint4* kr = reinterpret_cast<const uint4*>(sk + min(lane, nt - 1) * RS + w * 16);
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const uint4 kv = kr[i];
                const uint32_t wd[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const Acc k0 = (Acc)h2f((uint16_t)wd[e >> 1]), k1 = (Acc)h2f((uint16_t)(wd[e >> 1] >> 16));
#pragma unroll
                    for (int j = 0; j < HPW; j++) {
                        s0[j] = fma(sq[j][w * 16 + i * 8 + e], k0, s0[j]);
                        s1[j] = fma(sq[j][w * 16 + i * 8 + e + 1], k1, s1[j]);
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < HPW; j++) ss[j][w][lane] = s0[j] + s1[j];
        }
        __syncthreads();
        if (w < HPW) {   // wave j: head h0 + j
            Acc s = ss[w][0][lane];
#pragma unroll
            for (int v = 1; v < NW; v++) s += ss[w][v][lane];
            const Acc p = lane < nt ? acc_exp<Acc>(s * scale) : (Acc)0;
            sp[w][lane] = p;
            l += wave_sum(p);
        }
        __syncthreads();
        // p.V: dimensions 2*lane, 2*lane + 1 over positions t0 + 8w .. t0 + 8w + 7
#pragma unroll
        for (int u = 0; u < kAttnChunk / NW; u++) {
            const int t = w * (kAttnChunk / NW) + u;
            if (t < nt) {
                const uint32_t vw = *reinterpret_cast<const uint32_t*>(sv + t * RS + 2 * lane);
                const Acc v0 = (Acc)h2f((uint16_t)vw), v1 = (Acc)h2f((uint16_t)(vw >> 16));
#pragma unroll
                for (int j = 0; j < HPW; j++) {
                    const Acc pt = sp[j][t];
                    o[j][0] = fma(pt, v0, o[j][0]);
                    o[j][1] = fma(pt, v1, o[j][1]);
                }
            }
        }
        __syncthreads();   // the LDS rows and p are read no more in this chunk
    }
#pragma unroll
    for (int j = 0; j < HPW; j++) {
        so[w][j][2 * lane] = o[j][0];
        so[w][j][2 * lane + 1] = o[j][1];
    }
    if (lane == 0 && w < HPW) sl[w] = (double)l;
    __syncthreads();
    // threads 0 .. HPW*128 - 1: head h0 + tid/128, dimension tid%128, the
    // waves' sums in wave order
    const int oj = tid / HD, od = tid % HD;
    Acc ot = (Acc)0;
    if (tid < HPW * HD) {
        ot = so[0][oj][od];
#pragma unroll
        for (int v = 1; v < NW; v++) ot += so[v][oj][od];
    }
    if (!a.out && ng <= a.atomic_splits) {
        // each run adds its sums into the accumulators (zero on entry) with
        // fp64 atomics, which the launch's end makes visible to the o
        // projection's walk; no partials, no arrival, no last run
        double* O = reinterpret_cast<double*>(a.acc);
        if (tid < HPW * HD) atomicAdd(O + (size_t)(h0 + oj) * HD + od, (double)ot);
        if (tid >= HPW * HD && tid < HPW * HD + HPW)
            atomicAdd(O + (size_t)a.n_heads * HD + h0 + (tid - HPW * HD), sl[tid - HPW * HD]);
        return;
    }
    // each head's sums of the run go to its own slot of the partials (no two
    // runs add to one address): o at 0..127, the softmax sum at 128.  The
    // exchanges return the old values and the run waits for them before it
    // arrives (at the counter of its first head), so all are performed where
    // the last run's atomic loads read them.
    constexpr int PS = kAttnPartStride;
    double* part = reinterpret_cast<double*>(a.part);
    if (tid < HPW * (HD + 1)) {
        const int j = tid < HPW * HD ? oj : tid - HPW * HD, e = tid < HPW * HD ? od : HD;
        const double v = tid < HPW * HD ? (double)ot : sl[j];
        double* mine = part + ((size_t)(h0 + j) * gridDim.y + grp) * PS;
        const unsigned long long sink = __hip_atomic_exchange(reinterpret_cast<unsigned long long*>(mine + e),
                                                              (unsigned long long)__double_as_longlong(v),
                                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("" ::"v"(sink));
    }
    __syncthreads();
    if (tid == 0)
        s_last = __hip_atomic_fetch_add(a.head_ctr + h0, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (uint32_t)(ng - 1);
    __syncthreads();
    if (!s_last) return;
    // the last run of these heads: the sums over the runs, in run order, of
    // o (threads 0 .. HPW*128 - 1) and l (the next HPW threads); at most
    // kAttnGroups loads each
    double to = 0.0;
    const bool has = tid < HPW * (HD + 1);
    const int tj = tid < HPW * HD ? oj : tid - HPW * HD, te = tid < HPW * HD ? od : HD;
    if (has) {
        const double* first = part + (size_t)(h0 + tj) * gridDim.y * PS;
        double vo[kAttnGroups];
#pragma unroll
        for (int u = 0; u < kAttnGroups; u++)
            vo[u] = u < ng ? acc_peek(const_cast<double*>(first) + (size_t)u * PS + te) : 0.0;
#pragma unroll
        for (int u = 0; u < kAttnGroups; u++) to += vo[u];
    }
    if (has && te == HD) sl[tj] = to;
    if (a.out) {
        __syncthreads();
        if (tid < HPW * HD) a.out[(size_t)(h0 + oj) * HD + od] = (float)(to / sl[oj]);
    } else {
        double* O = reinterpret_cast<double*>(a.acc);
        if (tid < HPW * HD) O[(size_t)(h0 + oj) * HD + od] = to;
        if (has && te == HD) O[(size_t)a.n_heads * HD + h0 + tj] = to;
    }
    if (tid == 0) a.head_ctr[h0] = 0u;
}

// ---------------------------------------------------------------- embed ---
__global__ void k_embed(const uint16_t* __restrict__ table, int cols, int vocab,
                        const int* __restrict__ tok_p, float* __restrict__ out)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int tok = *tok_p;
    if (i >= cols) return;
    out[i] = (tok >= 0 && tok < vocab) ? h2f(table[(size_t)tok * cols + i]) : 0.0f;
}

// --------------------------------------------------------------- argmax ---
// first index of the maximum (std::max_element, test_generation.cpp:235)
__global__ __launch_bounds__(1024) void k_argmax(const float* __restrict__ v, int n,
                                                 int* __restrict__ out, int* __restrict__ pos_inc,
                                                 int* __restrict__ hist, int hist_len)
{
    __shared__ float sv[16];
    __shared__ int si[16];
    const int tid = threadIdx.x;
    float bv = -INFINITY;
    int bi = n;   // sentinel: larger than any index
    for (int i = tid; i < n; i += 1024) {
        const float x = v[i];
        if (x > bv || (x == bv && i < bi)) {
            bv = x;
            bi = i;
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if ((tid & 63) == 0) {
        sv[tid >> 6] = bv;
        si[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 16; w++)
            if (sv[w] > bv || (sv[w] == bv && si[w] < bi)) {
                bv = sv[w];
                bi = si[w];
            }
        const int tok = bi < n ? bi : 0;
        out[0] = tok;
        if (pos_inc) {
            const int np = pos_inc[0] + 1;
            if (hist && np >= 0 && np < hist_len) hist[np] = tok;
            pos_inc[0] = np;
        }
    }
}

// ------------------------------------------------------------------ host ---

template <int PER>
static int rmsnorm_per(Ctx* c, float* h, const float* delta, const uint16_t* gain, float eps, float* out)
{
    return launch(c, delta ? "add_rmsnorm" : "rmsnorm", k_rmsnorm<PER>, dim3(1), dim3(256), 0, h, delta, gain, eps,
                  out);
}

int rmsnorm(Ctx* c, float* h, const float* delta, const uint16_t* gain, int n, float eps, float* out)
{
    IAM_REQUIRE(n % 1024 == 0 && n >= 1024 && n <= 256 * kNormMaxPer,
                "rmsnorm: n must be a multiple of 1024 in [1024, 16384]");
    IAM_REQUIRE(((uintptr_t)h & 15) == 0 && ((uintptr_t)out & 15) == 0 && ((uintptr_t)delta & 15) == 0 &&
                    ((uintptr_t)gain & 7) == 0,
                "rmsnorm: vectors must be 16-byte aligned and the gain 8-byte aligned");
    switch (n / 256) {
        case 4: return rmsnorm_per<4>(c, h, delta, gain, eps, out);
        case 8: return rmsnorm_per<8>(c, h, delta, gain, eps, out);
        case 12: return rmsnorm_per<12>(c, h, delta, gain, eps, out);
        case 16: return rmsnorm_per<16>(c, h, delta, gain, eps, out);
        case 20: return rmsnorm_per<20>(c, h, delta, gain, eps, out);
        case 24: return rmsnorm_per<24>(c, h, delta, gain, eps, out);
        case 28: return rmsnorm_per<28>(c, h, delta, gain, eps, out);
        case 32: return rmsnorm_per<32>(c, h, delta, gain, eps, out);
        case 36: return rmsnorm_per<36>(c, h, delta, gain, eps, out);
        case 40: return rmsnorm_per<40>(c, h, delta, gain, eps, out);
        case 44: return rmsnorm_per<44>(c, h, delta, gain, eps, out);
        case 48: return rmsnorm_per<48>(c, h, delta, gain, eps, out);
        case 52: return rmsnorm_per<52>(c, h, delta, gain, eps, out);
        case 56: return rmsnorm_per<56>(c, h, delta, gain, eps, out);
        case 60: return rmsnorm_per<60>(c, h, delta, gain, eps, out);
        default: return rmsnorm_per<64>(c, h, delta, gain, eps, out);
    }
}

int resnorm(Ctx* c, const float* h, const void* delta_acc, float* h_out, const uint16_t* gain, int n, float eps,
            float* out)
{
    IAM_REQUIRE(n % 1024 == 0 && n >= 1024 && n <= 256 * kNormMaxPer,
                "resnorm: n must be a multiple of 1024 in [1024, 16384]");
    return launch(c, "resnorm", k_resnorm<double>, dim3(1), dim3(256), 0, h, (const double*)delta_acc, h_out, gain,
                  eps, n, out);
}

int add(Ctx* c, const float* a, const float* b, int n, float* out)
{
    return launch(c, "add32", k_add, dim3((n + 255) / 256), dim3(256), 0, a, b, n, out);
}

int silu_mul(Ctx* c, const float* g, const float* u, int n, float* out)
{
    return launch(c, "silu_mul", k_silu_mul, dim3((n + 255) / 256), dim3(256), 0, g, u, n, out);
}

int rope_kv(Ctx* c, const float* q, const float* k, const float* v, const float* table, const int* pos,
            int n_heads, int n_kv, int hd, int max_ctx, float* q_out, uint16_t* kc, uint16_t* vc)
{
    const int n = (n_heads + 2 * n_kv) * hd;
    return launch(c, "rope_kv_append", k_rope_kv, dim3((n + 255) / 256), dim3(256), 0, q, k, v, table, pos,
                  n_heads, n_kv, hd, max_ctx, q_out, kc, vc);
}

size_t attention_acc_words(int n_heads) { return (size_t)n_heads * 128 + (size_t)n_heads; }

size_t attention_part_words(int n_heads, int n_kv, int max_ctx)
{
    (void)n_kv;
    return (size_t)n_heads * (size_t)attn_runs(max_ctx) * kAttnPartStride;
}

int attention_launch(Ctx* c, const AttnLaunch& L)
{
    const int n_split = (L.max_ctx + kAttnChunk - 1) / kAttnChunk;
    IAM_REQUIRE(n_split <= kMaxAttnSplits, "attention: max_ctx above 8192");
    IAM_REQUIRE(L.part && L.head_ctr && (L.out || L.acc), "attention: missing scratch");
    AttnArgs a{};
    a.q = L.q;
    a.qkv_acc = L.qkv_acc;
    a.rope = L.rope;
    a.kc = L.kc;
    a.vc = L.vc;
    a.pos = L.pos;
    a.n_heads = L.n_heads;
    a.n_kv = L.n_kv;
    a.max_ctx = L.max_ctx;
    a.acc = L.acc;
    a.part = L.part;
    a.out = L.out;
    a.head_ctr = L.head_ctr;
    a.zero_p = L.zero_p;
    a.zero_n = L.zero_n;
    a.atomic_splits = L.acc && !L.out ? L.atomic_splits : 0;
    a.kv_copies = L.kv_copies;
    IAM_REQUIRE(L.n_heads <= kAttnMaxHeads, "attention: at most 512 query heads");
    // two query heads of one KV head per workgroup where the KV heads' query
    // heads pair up (each K and V value converted once for both): for 32
    // heads at most 32 runs x 16 workgroups, two resident per CU
    const bool pair = (L.n_heads / L.n_kv) % 2 == 0;
    const dim3 grid(L.n_heads / (pair ? 2 : 1), attn_runs(L.max_ctx)), block(kAttnThreads);
    const double sd = 1.0 / std::sqrt(128.0);
    const float sf = 1.0f / std::sqrt(128.0f);
    if (c->acc64) return pair ? launch(c, "attention", k_attn<double, 2>, grid, block, 0, a, sd)
                              : launch(c, "attention", k_attn<double, 1>, grid, block, 0, a, sd);
    return pair ? launch(c, "attention", k_attn<float, 2>, grid, block, 0, a, sf)
                : launch(c, "attention", k_attn<float, 1>, grid, block, 0, a, sf);
}

int embed(Ctx* c, const uint16_t* table, int cols, int vocab, const int* tok, float* out)
{
    return launch(c, "embed_gather", k_embed, dim3((cols + 255) / 256), dim3(256), 0, table, cols, vocab, tok,
                  out);
}

int argmax(Ctx* c, const float* v, int n, int* out, int* pos_inc, int* hist, int hist_len)
{
    return launch(c, "argmax", k_argmax, dim3(1), dim3(1024), 0, v, n, out, pos_inc, hist, hist_len);
}

}  // namespace iam

using namespace iam;

static int attn_shape_ok(int n_heads, int n_kv, int head_dim, int max_ctx)
{
    IAM_REQUIRE(head_dim == 128, "attention: head_dim must be 128");
    IAM_REQUIRE(n_kv >= 1 && n_heads >= n_kv && n_heads % n_kv == 0 && n_heads / n_kv <= kAttnMaxRep,
                "attention: n_heads must be a multiple of n_kv with at most 8 query heads per KV head");
    IAM_REQUIRE(max_ctx >= 1 && max_ctx <= kMaxAttnSplits * kAttnChunk, "attention: max_ctx must be in [1, 8192]");
    return IAM_OK;
}

extern "C" {

int iam_rmsnorm_gain(iam_ctx* c, const float* in, const uint16_t* gain, int n, float eps, float* out)
{
    if (!c || !in || !gain || !out) return fail(IAM_E_INVALID, "rmsnorm: null argument");
    IAM_REQUIRE(n > 0 && n % 1024 == 0, "rmsnorm: n must be a positive multiple of 1024");
    IAM_TRY(check_dev_range(c, in, (size_t)n * 4, "rmsnorm in"));
    IAM_TRY(check_dev_range(c, gain, (size_t)n * 2, "rmsnorm gain"));
    IAM_TRY(check_dev_range(c, out, (size_t)n * 4, "rmsnorm out"));
    return rmsnorm(c, const_cast<float*>(in), nullptr, gain, n, eps, out);
}

int iam_add_rmsnorm_gain(iam_ctx* c, float* h, const float* delta, const uint16_t* gain, int n, float eps,
                         float* out)
{
    if (!c || !h || !delta || !gain || !out) return fail(IAM_E_INVALID, "add_rmsnorm: null argument");
    IAM_REQUIRE(n > 0 && n % 1024 == 0, "add_rmsnorm: n must be a positive multiple of 1024");
    IAM_TRY(check_dev_range(c, h, (size_t)n * 4, "add_rmsnorm h"));
    IAM_TRY(check_dev_range(c, delta, (size_t)n * 4, "add_rmsnorm delta"));
    IAM_TRY(check_dev_range(c, gain, (size_t)n * 2, "add_rmsnorm gain"));
    IAM_TRY(check_dev_range(c, out, (size_t)n * 4, "add_rmsnorm out"));
    return rmsnorm(c, h, delta, gain, n, eps, out);
}

int iam_add(iam_ctx* c, const float* a, const float* b, int n, float* out)
{
    if (!c || !a || !b || !out) return fail(IAM_E_INVALID, "add: null argument");
    IAM_REQUIRE(n >= 0, "add: negative n");
    IAM_TRY(check_dev_range(c, a, (size_t)n * 4, "add a"));
    IAM_TRY(check_dev_range(c, b, (size_t)n * 4, "add b"));
    IAM_TRY(check_dev_range(c, out, (size_t)n * 4, "add out"));
    return add(c, a, b, n, out);
}

int iam_silu_mul(iam_ctx* c, const float* g, const float* u, int n, float* out)
{
    if (!c || !g || !u || !out) return fail(IAM_E_INVALID, "silu_mul: null argument");
    IAM_REQUIRE(n >= 0, "silu_mul: negative n");
    IAM_TRY(check_dev_range(c, g, (size_t)n * 4, "silu gate"));
    IAM_TRY(check_dev_range(c, u, (size_t)n * 4, "silu up"));
    IAM_TRY(check_dev_range(c, out, (size_t)n * 4, "silu out"));
    return silu_mul(c, g, u, n, out);
}

int iam_rope_table(double theta, int head_dim, int max_pos, float* table)
{
    if (!table || head_dim <= 0 || head_dim % 2 || max_pos <= 0)
        return fail(IAM_E_INVALID, "rope_table: bad argument");
    // attention.hpp:213-219: freq in double then float; angle = pos * freq in
    // float; cos/sin of the float angle
    const int half = head_dim / 2;
    for (int pos = 0; pos < max_pos; pos++) {
        for (int i = 0; i < half; i++) {
            double exponent = (2.0 * i) / head_dim;
            float freq = (float)(1.0f / std::pow(theta, exponent));
            float angle = (float)pos * freq;
            table[((size_t)pos * half + i) * 2 + 0] = std::cos(angle);
            table[((size_t)pos * half + i) * 2 + 1] = std::sin(angle);
        }
    }
    return IAM_OK;
}

int iam_rope(iam_ctx* c, const float* in, const float* table, const int* pos, int n_heads, int head_dim,
             float* out)
{
    if (!c || !in || !table || !pos || !out) return fail(IAM_E_INVALID, "rope: null argument");
    IAM_REQUIRE(n_heads > 0 && head_dim > 0 && head_dim % 2 == 0, "rope: bad shape");
    const size_t n = (size_t)n_heads * head_dim;
    IAM_TRY(check_dev_range(c, in, n * 4, "rope in"));
    IAM_TRY(check_dev_range(c, out, n * 4, "rope out"));
    IAM_TRY(check_dev_range(c, pos, 4, "rope pos"));
    // the table must hold whole rows; the kernel ignores positions past it
    auto it = c->allocs.upper_bound((uintptr_t)table);
    IAM_REQUIRE(it != c->allocs.begin(), "rope: table not allocated by this context");
    --it;
    const size_t avail = it->first + it->second - (uintptr_t)table;
    const int max_pos = (int)(avail / ((size_t)head_dim * 4));
    IAM_REQUIRE(max_pos >= 1, "rope: table too small");
    return launch(c, "rope", k_rope, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, in, table, pos, n_heads,
                  head_dim, max_pos, out);
}

int iam_rope_kv_append(iam_ctx* c, const float* q, const float* k, const float* v, const float* table,
                       const int* pos, int n_heads, int n_kv, int head_dim, int max_ctx, float* q_out,
                       uint16_t* kc, uint16_t* vc)
{
    if (!c || !q || !k || !v || !table || !pos || !q_out || !kc || !vc)
        return fail(IAM_E_INVALID, "rope_kv_append: null argument");
    IAM_REQUIRE(n_heads > 0 && n_kv > 0 && head_dim > 0 && head_dim % 2 == 0 && max_ctx > 0,
                "rope_kv_append: bad shape");
    const size_t nq = (size_t)n_heads * head_dim, nk = (size_t)n_kv * head_dim;
    IAM_TRY(check_dev_range(c, q, nq * 4, "rope_kv q"));
    IAM_TRY(check_dev_range(c, k, nk * 4, "rope_kv k"));
    IAM_TRY(check_dev_range(c, v, nk * 4, "rope_kv v"));
    IAM_TRY(check_dev_range(c, q_out, nq * 4, "rope_kv q_out"));
    IAM_TRY(check_dev_range(c, table, (size_t)max_ctx * head_dim * 4, "rope_kv table"));
    IAM_TRY(check_dev_range(c, kc, (size_t)max_ctx * nk * 2, "rope_kv kcache"));
    IAM_TRY(check_dev_range(c, vc, (size_t)max_ctx * nk * 2, "rope_kv vcache"));
    IAM_TRY(check_dev_range(c, pos, 4, "rope_kv pos"));
    return rope_kv(c, q, k, v, table, pos, n_heads, n_kv, head_dim, max_ctx, q_out, kc, vc);
}

int iam_attention_decode(iam_ctx* c, const float* q, const uint16_t* kc, const uint16_t* vc, const int* pos,
                         int n_heads, int n_kv, int head_dim, int max_ctx, float* out)
{
    if (!c || !q || !kc || !vc || !pos || !out) return fail(IAM_E_INVALID, "attention: null argument");
    IAM_TRY(attn_shape_ok(n_heads, n_kv, head_dim, max_ctx));
    const size_t nk = (size_t)n_kv * head_dim;
    IAM_TRY(check_dev_range(c, q, (size_t)n_heads * head_dim * 4, "attention q"));
    IAM_TRY(check_dev_range(c, kc, (size_t)max_ctx * nk * 2, "attention kcache"));
    IAM_TRY(check_dev_range(c, vc, (size_t)max_ctx * nk * 2, "attention vcache"));
    IAM_TRY(check_dev_range(c, out, (size_t)n_heads * head_dim * 4, "attention out"));
    IAM_TRY(check_dev_range(c, pos, 4, "attention pos"));
    IAM_TRY(ensure_attn_scratch(c, attention_part_words(n_heads, n_kv, max_ctx), n_heads));
    AttnLaunch L{};
    L.q = q;
    L.kc = const_cast<uint16_t*>(kc);
    L.vc = const_cast<uint16_t*>(vc);
    L.pos = pos;
    L.n_heads = n_heads;
    L.n_kv = n_kv;
    L.max_ctx = max_ctx;
    L.part = c->attn_acc;
    L.out = out;
    L.head_ctr = c->attn_ctr;
    return attention_launch(c, L);
}

int iam_embed_gather(iam_ctx* c, const uint16_t* table, int cols, int vocab, const int* tok, float* out)
{
    if (!c || !table || !tok || !out) return fail(IAM_E_INVALID, "embed: null argument");
    IAM_REQUIRE(cols > 0 && vocab > 0, "embed: bad shape");
    IAM_TRY(check_dev_range(c, table, (size_t)cols * vocab * 2, "embed table"));
    IAM_TRY(check_dev_range(c, out, (size_t)cols * 4, "embed out"));
    IAM_TRY(check_dev_range(c, tok, 4, "embed token"));
    return embed(c, table, cols, vocab, tok, out);
}

int iam_argmax(iam_ctx* c, const float* v, int n, int* out)
{
    if (!c || !v || !out) return fail(IAM_E_INVALID, "argmax: null argument");
    IAM_REQUIRE(n > 0, "argmax: n must be positive");
    IAM_TRY(check_dev_range(c, v, (size_t)n * 4, "argmax v"));
    IAM_TRY(check_dev_range(c, out, 4, "argmax out"));
    return argmax(c, v, n, out, nullptr);
}

}  // extern "C"
