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
// Decode attention over an fp16 GQA cache, split over the context.
// Workgroup (kv head, split) handles kAttnChunk = 64 positions for the rep =
// n_heads/n_kv query heads that read this KV head (repeat4x32,
// aux.cl:266-275, without materialising the repeat): wave r is query head
// kvh*rep + r % rep and half r / rep of the head dimension, lane i position
// t0 + i.  Each lane computes its position's half dot product (dotSetScore2,
// aux.cl:497-540, s = q.k / sqrt(hd)) with q broadcast from LDS, and the
// halves are added through LDS; p = exp(s) (sum_of_exps32_mx /
// softmax_add32_mx, aux.cl:204-225: the reference's softmax has no maximum
// subtracted, so the splits' sums add up directly); then lane (g, j)
// accumulates 8 dimensions of the wave's half of sum p*V over every eighth
// position.  The splits' sums p*V (rep heads x 128) and sums of p then
// meet in o and l for the consumer (the o projection's walk, which divides
// x = o / l), or, for the standalone call, out = o / l (sumScores32,
// aux.cl:370-384).  In the model, while a KV head has at most
// atomic_splits splits, each split adds its sums into o and l with fp64
// atomics (the sums within an fp64 rounding of the exact ones, whatever the
// order).  Otherwise each split writes its sums to its own slot of the
// partials with atomic exchanges, waits for them to be performed and
// arrives at its KV head's counter; the last split to arrive adds the slots
// in split order (no two splits add to one address, so the sums do not
// depend on arrival order) and writes o and l, or out.  The
// split's K and V rows are loaded once per workgroup, 16 bytes per thread,
// into LDS.  With the projection accumulators as input the workgroup also
// applies RoPE to q and k (rope_mx, aux.cl:227-248, table row of the
// position) and the split holding the position appends the new K and V rows
// to the cache (attention.hpp:281-309) and uses them from LDS.  Acc = double
// evaluates every product (exact: fp32 x fp16), exponential and sum in fp64
// (a score above log(DBL_MAX) ~ 709.78 overflows, as the reference's fp32
// exp does above 88.72); Acc = float in fp32.
constexpr int kAttnChunk = 64;
constexpr int kAttnMaxRep = 8;
constexpr int kMaxAttnSplits = 128;   // max_ctx up to 8192
// doubles per split and KV head in the partials: o of rep heads, the rep
// softmax sums, padded to 64 bytes
__host__ __device__ constexpr int attn_part_stride(int rep) { return rep * 128 + 8; }

// v + v of lane l ^ 8 (a DPP rotation by 8 within each row of 16 lanes)
__device__ __forceinline__ double xsum8(double v) { return v + dpp_d<0x128>(v, v); }
__device__ __forceinline__ float xsum8(float v) { return v + dpp_f<0x128>(v, v); }

// v + v of lane l ^ M for M = 16 or 32: v_permlane{16,32}_swap with both
// operands v returns (v of lane l & ~M, v of lane l | M) in every lane
template <int M>
__device__ __forceinline__ void swap_pair(uint32_t w, uint32_t& lo_lane, uint32_t& hi_lane)
{
    static_assert(M == 16 || M == 32, "16 or 32");
    if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(w, w, false, false);
        lo_lane = r[0];
        hi_lane = r[1];
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(w, w, false, false);
        lo_lane = r[0];
        hi_lane = r[1];
    }
}
template <int M>
__device__ __forceinline__ double xsum_swap(double v)
{
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    uint32_t l0, l1, h0, h1;
    swap_pair<M>((uint32_t)b, l0, l1);
    swap_pair<M>((uint32_t)(b >> 32), h0, h1);
    return __longlong_as_double((long long)(((unsigned long long)h0 << 32) | l0)) +
           __longlong_as_double((long long)(((unsigned long long)h1 << 32) | l1));
}
template <int M>
__device__ __forceinline__ float xsum_swap(float v)
{
    uint32_t a, b;
    swap_pair<M>(__float_as_uint(v), a, b);
    return __uint_as_float(a) + __uint_as_float(b);
}

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
    void* acc;               // o [n_heads][128], then l [n_heads] (fp64): written by the last
                             // split of each KV head (model mode)
    void* part;              // the splits' partial sums [n_kv][splits][attn_part_stride(rep)] (fp64)
    float* out;              // standalone: out = o / l, stored by the last split of each KV head
    uint32_t* head_ctr;      // [n_kv] arrival counters, zero on entry (left zero)
    void* zero_p;            // accumulator words cleared by this launch
    int zero_n;
    int atomic_splits;       // model: splits per KV head up to which o and l are added with atomics
};

// LDS copies of the split's K and V rows.  A 16-byte LDS access is served 16
// lanes at a time over 64 banks of 4 bytes.  K rows are read one row per
// lane (the dot products): 128 fp16 + 8 of padding (68 words) puts 16
// consecutive rows on 16 disjoint groups of 4 banks.  V rows are read 8
// lanes per row (p.V): 128 fp16 + 64 of padding (96 words, 32 banks apart)
// puts the two rows of a 16-lane group on disjoint halves of the banks.
constexpr int kAttnRowStride = 128 + 8;
constexpr int kAttnVStride = 128 + 64;
static_assert(kAttnChunk * kAttnRowStride * 2 >= kMaxAttnSplits * kAttnMaxRep * 8,
              "the K rows' LDS holds the softmax-sum partials of the last split");

template <typename Acc>
__global__ __launch_bounds__(128 * kAttnMaxRep) void k_attn(AttnArgs a, Acc scale)
{
#pragma clang fp contract(off)
    constexpr int HD = 128, RS = kAttnRowStride, VS = kAttnVStride, DH = HD / 2;
    __shared__ __align__(16) uint16_t sk[kAttnChunk * RS];
    __shared__ __align__(16) uint16_t sv[kAttnChunk * VS];
    __shared__ Acc sq[kAttnMaxRep][HD];
    __shared__ Acc ss[2][kAttnMaxRep][kAttnChunk];          // half-dot products
    __shared__ Acc sp[2 * kAttnMaxRep][kAttnChunk];         // p, one copy per wave
    __shared__ double sl[kAttnMaxRep];
    __shared__ int s_last;
    const int rep = a.n_heads / a.n_kv;
    const int nthr = 128 * rep;
    zero_share<double>(a.zero_p, a.zero_n, nthr);
    const int kvh = blockIdx.x;
    const int split = blockIdx.y;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int r = tid >> 6;
    const int hr = r % rep, hf = r / rep;
    const int pos = *a.pos;
    const int n_tok = min(pos + 1, a.max_ctx);
    const int t0 = split * kAttnChunk;
    const int nt = min(kAttnChunk, max(0, n_tok - t0));
    if (nt == 0) return;   // past the context: neither written nor counted
    const bool pos_ok = pos >= 0 && pos < a.max_ctx;
    const int h = kvh * rep + hr;
    const double* A = reinterpret_cast<const double*>(a.qkv_acc);
    const bool fresh = A && pos_ok && pos >= t0 && pos < t0 + kAttnChunk;   // this split holds the new row
    float c = 1.0f, sn = 0.0f;
    if (A && pos_ok) {
        c = a.rope[(size_t)pos * HD + 2 * lane];
        sn = a.rope[(size_t)pos * HD + 2 * lane + 1];
    }
    // q of dimension hf*64 + lane
    float qv;
    if (A) {
        const float lo = (float)A[(size_t)h * HD + lane], hi = (float)A[(size_t)h * HD + DH + lane];
        qv = hf == 0 ? __fsub_rn(__fmul_rn(lo, c), __fmul_rn(hi, sn))    // rope_mx: d < 64
                     : __fadd_rn(__fmul_rn(hi, c), __fmul_rn(lo, sn));   // d >= 64
    } else {
        qv = a.q[(size_t)h * HD + hf * DH + lane];
    }
    // the split's K and V rows (the fresh row comes from the accumulators)
    const int pieces = nt * (HD / 8);
    for (int b0 = 0; b0 < pieces; b0 += 4 * nthr) {
        uint4 kq[4], vq[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int idx = min(b0 + u * nthr + tid, pieces - 1);
            const size_t g = ((size_t)(t0 + (idx >> 4)) * a.n_kv + kvh) * HD + (idx & 15) * 8;
            kq[u] = *reinterpret_cast<const uint4*>(a.kc + g);
            vq[u] = *reinterpret_cast<const uint4*>(a.vc + g);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int idx = b0 + u * nthr + tid;
            if (idx < pieces && !(fresh && t0 + (idx >> 4) == pos)) {
                *reinterpret_cast<uint4*>(sk + (idx >> 4) * RS + (idx & 15) * 8) = kq[u];
                *reinterpret_cast<uint4*>(sv + (idx >> 4) * VS + (idx & 15) * 8) = vq[u];
            }
        }
    }
    if (fresh && r < 2) {
        // wave 0: k after RoPE; wave 1: v; both rounded to fp16 into the
        // cache row and the LDS row
        const int nq = a.n_heads * HD, nk = a.n_kv * HD;
        const size_t base = (size_t)(r == 0 ? nq : nq + nk) + (size_t)kvh * HD;
        const float lo = (float)A[base + lane], hi = (float)A[base + DH + lane];
        float o0 = lo, o1 = hi;
        if (r == 0) {
            o0 = __fsub_rn(__fmul_rn(lo, c), __fmul_rn(hi, sn));
            o1 = __fadd_rn(__fmul_rn(hi, c), __fmul_rn(lo, sn));
        }
        const uint16_t h0 = __half_as_ushort(__float2half_rn(o0)), h1 = __half_as_ushort(__float2half_rn(o1));
        uint16_t* crow = (r == 0 ? a.kc : a.vc) + ((size_t)pos * a.n_kv + kvh) * HD;
        crow[lane] = h0;
        crow[DH + lane] = h1;
        uint16_t* lrow = r == 0 ? sk + (pos - t0) * RS : sv + (pos - t0) * VS;
        lrow[lane] = h0;
        lrow[DH + lane] = h1;
    }
    sq[hr][hf * DH + lane] = (Acc)qv;
    __syncthreads();
    // half dot product of position t0 + lane (four chains of 16 products,
    // dimensions 4m + c in chain c, then added pairwise), then the two halves
    // in order
    {
        Acc sc[4] = {(Acc)0, (Acc)0, (Acc)0, (Acc)0};
        const uint4* kr = reinterpret_cast<const uint4*>(sk + min(lane, nt - 1) * RS + hf * DH);
#pragma unroll
        for (int i = 0; i < DH / 8; i++) {
            const uint4 kv = kr[i];
            const uint32_t w[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
            for (int e = 0; e < 8; e++)
                sc[e & 3] = fma(sq[hr][hf * DH + i * 8 + e], (Acc)h2f((uint16_t)(w[e >> 1] >> ((e & 1) * 16))),
                                sc[e & 3]);
        }
        ss[hf][hr][lane] = (sc[0] + sc[1]) + (sc[2] + sc[3]);
    }
    __syncthreads();
    const Acc s = (ss[0][hr][lane] + ss[1][hr][lane]) * scale;
    const Acc p = lane < nt ? acc_exp<Acc>(s) : (Acc)0;
    const Acc l = wave_sum(p);
    sp[r][lane] = p;   // read back by this wave only: no barrier
    // sum of p * V over this half's dimensions: lane (g, j) takes dimensions
    // hf*64 + 8j..8j+7 of the positions g, g + 8, ...; the eight g partials
    // are added pairwise across lanes
    const int g = lane >> 3, j = lane & 7;
    Acc o[8];
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = (Acc)0;
#pragma unroll
    for (int u = 0; u < kAttnChunk / 8; u++) {
        const int i = g + 8 * u;
        if (i < nt) {
            const Acc pi = sp[r][i];
            const uint4 vv = *reinterpret_cast<const uint4*>(sv + i * VS + hf * DH + j * 8);
            const uint32_t w[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
            for (int e = 0; e < 8; e++)
                o[e] = fma(pi, (Acc)h2f((uint16_t)(w[e >> 1] >> ((e & 1) * 16))), o[e]);
        }
    }
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = xsum_swap<32>(xsum_swap<16>(xsum8(o[e])));
    Acc og = o[0];   // lane (g, j): dimension hf*64 + j*8 + g
#pragma unroll
    for (int e = 1; e < 8; e++) og = g == e ? o[e] : og;
    const int ns = (n_tok + kAttnChunk - 1) / kAttnChunk;   // the KV head's splits
    if (!a.out && ns <= a.atomic_splits) {
        // few splits: each adds its sums into the accumulators (zero on
        // entry) with fp64 atomics, which the launch's end makes visible to
        // the o projection's walk; no partials, no arrival, no last split
        double* O = reinterpret_cast<double*>(a.acc);
        atomicAdd(O + (size_t)h * HD + hf * DH + j * 8 + g, (double)og);
        if (hf == 0 && lane == 0) atomicAdd(O + (size_t)a.n_heads * HD + h, (double)l);
        return;
    }
    // the split's partial sums go to its own slot of the partials (no two
    // splits add to one address): lane (g, j) holds dimension
    // hf*64 + j*8 + g at slot position hr*128 + hf*64 + g*8 + j, so a wave
    // writes 64 consecutive values; then the softmax sums.  The exchanges
    // return the old values and the split waits for them before it arrives,
    // so all are performed where the last split's atomic loads read them.
    const int PS = attn_part_stride(rep);
    double* part = reinterpret_cast<double*>(a.part);
    double* mine = part + ((size_t)kvh * gridDim.y + split) * PS;
    unsigned long long sink = __hip_atomic_exchange(
        reinterpret_cast<unsigned long long*>(mine + hr * HD + hf * DH + lane),
        (unsigned long long)__double_as_longlong((double)og), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (hf == 0 && lane == 0)
        sink += __hip_atomic_exchange(reinterpret_cast<unsigned long long*>(mine + rep * HD + hr),
                                      (unsigned long long)__double_as_longlong((double)l), __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("" ::"v"(sink));
    __syncthreads();
    if (tid == 0)
        s_last = __hip_atomic_fetch_add(a.head_ctr + kvh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (uint32_t)(ns - 1);
    __syncthreads();
    if (!s_last) return;
    // the last split of this KV head: the sums over the splits, in split
    // order, of o (rep heads x 128: one value per thread, 16 splits' loads
    // in flight) and l (thread t < rep * ns loads split t / rep's value of
    // head t % rep into LDS, where the first threads add them up)
    const double* first = part + (size_t)kvh * gridDim.y * PS;
    const bool has_lp = tid < rep * ns;
    const double lp = has_lp ? acc_peek(const_cast<double*>(first) + (size_t)(tid / rep) * PS + rep * HD + tid % rep)
                             : 0.0;
    double to = 0.0;
    for (int s0 = 0; s0 < ns; s0 += 16) {
        double vo[16];
#pragma unroll
        for (int u = 0; u < 16; u++)
            vo[u] = s0 + u < ns ? acc_peek(const_cast<double*>(first) + (size_t)(s0 + u) * PS + tid) : 0.0;
#pragma unroll
        for (int u = 0; u < 16; u++) to += vo[u];
    }
    double* s_lp = reinterpret_cast<double*>(sk);   // the K rows are read no more
    if (has_lp) s_lp[tid] = lp;
    __syncthreads();
    if (tid < rep) {
        double tl = 0.0;
        for (int sp_ = 0; sp_ < ns; sp_++) tl += s_lp[sp_ * rep + tid];
        sl[tid] = tl;
    }
    // slot position tid -> head and dimension
    const int hh = tid / HD, pp = tid % HD;
    const int d = (pp / DH) * DH + (pp % 8) * 8 + (pp % DH) / 8;
    const size_t oi = (size_t)(kvh * rep + hh) * HD + d;
    double* O = reinterpret_cast<double*>(a.acc);
    if (a.out) {
        __syncthreads();
        a.out[oi] = (float)(to / sl[hh]);
    } else {
        O[oi] = to;
        if (tid < rep) O[(size_t)a.n_heads * HD + kvh * rep + tid] = sl[tid];
    }
    if (tid == 0) a.head_ctr[kvh] = 0u;
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
    return (size_t)n_kv * (size_t)((max_ctx + kAttnChunk - 1) / kAttnChunk) * attn_part_stride(n_heads / n_kv);
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
    const dim3 grid(L.n_kv, n_split), block(128 * (L.n_heads / L.n_kv));
    if (c->acc64) return launch(c, "attention", k_attn<double>, grid, block, 0, a, 1.0 / std::sqrt(128.0));
    return launch(c, "attention", k_attn<float>, grid, block, 0, a, 1.0f / std::sqrt(128.0f));
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
    IAM_TRY(ensure_attn_scratch(c, attention_part_words(n_heads, n_kv, max_ctx), n_kv));
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
