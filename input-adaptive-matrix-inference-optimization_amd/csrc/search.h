// Cutoff search of findCutoffBinarySearch (bucketMul.cl:68-214) for one
// workgroup of 4 or 8 waves, resolved several bisection rounds at a time.
//
// The reference bisects [min, max] of the 4096 importances for at most 20
// rounds: it counts c = #(imp > bound), moves max (c < target) or min
// (otherwise) to the bound, and stops on c == target, max - min < 1e-5 or
// |maxCount - minCount| < 3, returning the tested bound (or, after 20
// rounds, the untested midpoint of the last bracket).  Every bound it can
// test in the next D rounds is a node of the depth-D tree of float midpoints
// of the current bracket, and every count it needs is a count of the
// importances above one of those nodes.  A stage therefore:
//   1. computes the 2^D leaf edges of that tree (each lane walks the
//      midpoint recurrence down to its leaves, in the reference's fp32
//      arithmetic, so the edges are the reference's bounds bit for bit);
//   2. bins the importances inside the bracket into the leaves (LDS
//      histogram, one per wave);
//   3. after one barrier, turns the histogram into the count above every
//      node (a suffix sum), finds the leaf the bisection ends in, and
//      evaluates the stop tests of its D rounds in parallel (lane l takes
//      round l); the first round that stops gives the cutoff.
// Otherwise the next stage continues from that leaf's bracket.  The tested
// bounds, counts, updates and stop decisions are those of the reference, so
// the cutoff is the same float; two stages cover typical inputs (about 12
// rounds), three the 20-round limit.
#pragma once

#include "wave.h"

namespace iam {

constexpr int kCutThreads = 256;              // threads holding importances
constexpr int kCutVPT = IAM_PROBES_COUNT / kCutThreads;   // 16 per thread
constexpr int kMaxDepth = 8;                  // rounds per stage
constexpr int kLeaves = 1 << kMaxDepth;

template <int NW>
struct SearchLds {
    float E[NW][kLeaves];            // leaf upper edges, one copy per wave
    uint32_t S[NW][kLeaves];         // counts above each leaf start, one copy per wave
    uint32_t H[2][4][kLeaves];       // histograms of the 4 value-holding waves, two stages
    float red[2 * NW];
};

__device__ __forceinline__ float uniform_f(float v)
{
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

__device__ __forceinline__ int uniform_i(int v) { return __builtin_amdgcn_readfirstlane(v); }

// (lo + hi) / 2.0f of bucketMul.cl:139, :190 (halving is exact, so * 0.5f
// gives the same float)
__device__ __forceinline__ float midpoint(float lo, float hi)
{
    return __fmul_rn(__fadd_rn(lo, hi), 0.5f);
}

// The cutoff of the 4096 importances held 16 per thread by the first 256
// threads (v; other threads' values are ignored).  Every thread returns it.
// Two barriers plus one per stage; on return the scratch may be reused
// after a further barrier.
template <int NW>
__device__ float search_cutoff(const float (&v)[kCutVPT], int quantile, SearchLds<NW>& L)
{
#pragma clang fp contract(off)
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const bool holder = tid < kCutThreads;

    float mn = 1e30f, mx = -1e30f;                     // bucketMul.cl:98-99
    if (holder) {
#pragma unroll
        for (int k = 0; k < kCutVPT; k++) {
            mn = fminf(mn, v[k]);
            mx = fmaxf(mx, v[k]);
        }
    }
    mn = wave_min(mn);
    mx = wave_max(mx);
    if (lane == 0) {
        L.red[wave] = mn;
        L.red[NW + wave] = mx;
    }
    __syncthreads();
    float gmin = 1e30f, gmax = -1e30f;
#pragma unroll
    for (int w = 0; w < NW; w++) {
        gmin = fminf(gmin, L.red[w]);
        gmax = fmaxf(gmax, L.red[NW + w]);
    }
    const int target = IAM_PROBES_COUNT - quantile;    // bucketMul.cl:81
    float minB = uniform_f(gmin), maxB = uniform_f(gmax);
    int minC = IAM_PROBES_COUNT, maxC = 0;             // bucketMul.cl:142-143
    int rounds = 0, buf = 0;
    float* E = L.E[wave];
    uint32_t* S = L.S[wave];
    for (;;) {
        const int D = min(kMaxDepth, 20 - rounds);
        const int NL = 1 << D;
        // 1. leaf edges: lane l takes leaves 4l .. 4l+3 (their paths share
        // all but the last two levels)
        if (4 * lane < NL || lane == 0) {
            float lo = minB, hi = maxB;
            const int pre = D >= 2 ? D - 2 : 0;
            for (int l = 0; l < pre; l++) {
                const float b = midpoint(lo, hi);
                if ((lane >> (pre - 1 - l)) & 1) lo = b;
                else hi = b;
            }
            float4 e;
            if (D >= 2) {
                const float mid = midpoint(lo, hi);
                e = make_float4(midpoint(lo, mid), mid, midpoint(mid, hi), hi);
            } else {
                e = make_float4(midpoint(lo, hi), hi, hi, hi);
            }
            *reinterpret_cast<float4*>(E + 4 * lane) = e;
        }
        // 2. histogram of the bracket (minB, maxB] over the leaves
        if (holder) {
            uint32_t* H = L.H[buf][wave];
            *reinterpret_cast<uint4*>(H + 4 * lane) = make_uint4(0u, 0u, 0u, 0u);
            // Binning by position: the edges lie within a small fraction of
            // a leaf of their dyadic positions when the bracket is wide
            // against the float spacing at maxB (and no midpoint sum
            // overflows), so the estimated leaf is off by at most one and one
            // comparison on each side fixes it; otherwise a binary search.
            const float w = __fsub_rn(maxB, minB);
            const bool guess = w > 0.0f && maxB < 1.0e38f && w > __fmul_rn(fmaxf(maxB, 1e-30f), 0.00025f);
            const float scale = guess ? __fdiv_rn((float)NL, w) : 0.0f;
            // every value gets a leaf (those outside the bracket are not
            // counted), so the LDS reads of all 16 go out together
            int g[kCutVPT];
            if (guess) {
                float eg[kCutVPT], em[kCutVPT];
#pragma unroll
                for (int k = 0; k < kCutVPT; k++) {
                    const float f = __fmul_rn(__fsub_rn(v[k], minB), scale);
                    g[k] = (int)fminf(fmaxf(f, 0.0f), (float)(NL - 1));   // NaN -> 0
                }
#pragma unroll
                for (int k = 0; k < kCutVPT; k++) {
                    eg[k] = E[g[k]];
                    em[k] = E[g[k] > 0 ? g[k] - 1 : 0];
                }
#pragma unroll
                for (int k = 0; k < kCutVPT; k++) {
                    if (g[k] < NL - 1 && eg[k] < v[k]) g[k]++;
                    else if (g[k] > 0 && em[k] >= v[k]) g[k]--;
                }
            } else {
#pragma unroll
                for (int k = 0; k < kCutVPT; k++) g[k] = 0;   // #(edges E[0 .. NL-2] below the value)
                for (int st = NL >> 1; st > 0; st >>= 1) {
                    float e[kCutVPT];
#pragma unroll
                    for (int k = 0; k < kCutVPT; k++) e[k] = E[min(g[k] + st - 1, NL - 2)];
#pragma unroll
                    for (int k = 0; k < kCutVPT; k++)
                        if (g[k] + st <= NL - 1 && e[k] < v[k]) g[k] += st;
                }
            }
#pragma unroll
            for (int k = 0; k < kCutVPT; k++)
                if (v[k] > minB && v[k] <= maxB) atomicAdd(H + g[k], 1u);
        }
        __syncthreads();
        // 3. S[j] = #(bracket values in leaves >= j), every wave for itself
        uint32_t c0, c1, c2, c3;
        {
            const uint4 h0 = *reinterpret_cast<const uint4*>(L.H[buf][0] + 4 * lane);
            const uint4 h1 = *reinterpret_cast<const uint4*>(L.H[buf][1] + 4 * lane);
            const uint4 h2 = *reinterpret_cast<const uint4*>(L.H[buf][2] + 4 * lane);
            const uint4 h3 = *reinterpret_cast<const uint4*>(L.H[buf][3] + 4 * lane);
            c0 = h0.x + h1.x + h2.x + h3.x;
            c1 = h0.y + h1.y + h2.y + h3.y;
            c2 = h0.z + h1.z + h2.z + h3.z;
            c3 = h0.w + h1.w + h2.w + h3.w;
        }
        const uint32_t s3 = c3, s2 = c2 + s3, s1 = c1 + s2, s0 = c0 + s1;
        const int incl = wave_incl_sum((int)s0);
        const uint32_t above = (uint32_t)(__builtin_amdgcn_readlane(incl, 63) - incl);   // lanes > this one
        const uint32_t S0 = s0 + above, S1 = s1 + above, S2 = s2 + above, S3 = s3 + above;
        *reinterpret_cast<uint4*>(S + 4 * lane) = make_uint4(S0, S1, S2, S3);
        // the leaf the rounds end in: count(imp > E[m-1]) = maxC + S[m] >=
        // target exactly for m <= js (going up the tree at that node)
        const int m0 = 4 * lane;
        int js = __popcll(__ballot(m0 >= 1 && m0 < NL && maxC + (int)S0 >= target)) +
                 __popcll(__ballot(m0 + 1 < NL && maxC + (int)S1 >= target)) +
                 __popcll(__ballot(m0 + 2 < NL && maxC + (int)S2 >= target)) +
                 __popcll(__ballot(m0 + 3 < NL && maxC + (int)S3 >= target));
        js = uniform_i(js);
        // the stop tests of rounds 0 .. D-1 of this stage (bucketMul.cl:178-200)
        bool stop = false;
        float tested = 0.0f;
        if (lane < D) {
            const int sh = D - lane;                     // the round's node covers 2^sh leaves
            const int half = 1 << (sh - 1);
            const int a = (js >> sh) << sh;
            const int m = a + half;
            tested = E[m - 1];
            const int c = maxC + (int)S[m];
            const int a1 = (js >> (sh - 1)) << (sh - 1);   // the bracket after the update
            const float lo = a1 == 0 ? minB : E[a1 - 1];
            const float hi = a1 + half == NL ? maxB : E[a1 + half - 1];
            const int lc = a1 == 0 ? minC : maxC + (int)S[a1];
            const int hc = a1 + half == NL ? maxC : maxC + (int)S[a1 + half];
            const int gap = hc - lc;
            stop = c == target || __fsub_rn(hi, lo) < 0.00001f || (gap < 0 ? -gap : gap) < 3;
        }
        const uint64_t sm = __ballot(stop);
        if (sm) return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tested), __ffsll((long long)sm) - 1));
        // continue from leaf js's bracket
        const float nlo = js == 0 ? minB : E[js - 1];
        const float nhi = js == NL - 1 ? maxB : E[js];
        const int nlc = js == 0 ? minC : maxC + (int)S[js];
        const int nhc = js == NL - 1 ? maxC : maxC + (int)S[js + 1];
        minB = uniform_f(nlo);
        maxB = uniform_f(nhi);
        minC = uniform_i(nlc);
        maxC = uniform_i(nhc);
        rounds += D;
        buf ^= 1;
        if (rounds >= 20) return midpoint(minB, maxB);   // bucketMul.cl:211-213: the untested midpoint
    }
}

}  // namespace iam
