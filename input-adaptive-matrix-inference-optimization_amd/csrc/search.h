// Cutoff search of findCutoffBinarySearch (bucketMul.cl:68-214) for one
// workgroup of 4 or 8 waves.
//
// The reference bisects [min, max] of the 4096 importances for at most 20
// rounds: it counts c = #(imp > bound), moves max (c < target) or min
// (otherwise) to the bound, and stops on c == target, max - min < 1e-5 or
// |maxCount - minCount| < 3, returning the tested bound (or, after 20
// rounds, the untested midpoint of the last bracket).  With u_j the j-th
// largest importance (NaN below every value: NaN > b is false),
// #(imp > b) >= j exactly when u_j > b.  So every decision of the reference
// follows from t = target and u_{t-2} .. u_{t+2}: the round moves max iff
// u_t <= b, the count equals t iff u_t > b >= u_{t+1}, and the bracket's
// counts differ by less than 3 only in cases that compare u_{t-2}, u_{t-1},
// u_{t+1}, u_{t+2} with its ends.  The search therefore
//   1. maps the importances to order-preserving 32-bit keys (NaN -> 0) and
//      reduces their min, max and count;
//   2. selects the key of rank a = min(t, #non-NaN) with a radix select:
//      digits of key - min from the top bit of max - min down, 8 bits a pass,
//      counted in per-wave LDS histograms (one barrier a pass; every wave
//      scans the summed histogram itself); a digit bin holding one key ends
//      it early.  Digits of the key's offset from the minimum spread a
//      heavy-tailed distribution over many bins (the float exponent is in
//      the top bits), which keeps LDS atomics on one address few;
//   3. one pass for the two nearest keys on either side of u_a (the counts
//      above and equal to it come out of the select): every rank within two
//      of t lies in that neighbourhood;
//   4. replays the reference's rounds in its fp32 arithmetic, lane r taking
//      round r, and returns the first round that stops, so the cutoff is the
//      reference's float bit for bit.
#pragma once

#include "wave.h"

namespace iam {

constexpr int kCutThreads = 256;              // threads of the standalone cutoff kernels
constexpr int kCutVPT = IAM_PROBES_COUNT / kCutThreads;   // 16 importances per thread there

template <int NW>
struct SearchLds {
    uint32_t H[2][NW][256];    // digit histograms of the waves, two passes
    uint32_t red[2][NW];       // key min - 1, key max per wave
    uint32_t nb[NW][4];        // per wave: the two smallest keys above u's bin, and of ~key below it
    uint32_t tie[NW];          // per wave: the largest key in u's bin
    float cut;                 // the cutoff (wave 0 writes it)
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

// order-preserving key of a float; NaN maps below every number (to 0, whose
// float, a NaN, compares like -inf in every v > b)
__device__ __forceinline__ uint32_t order_key(float f)
{
    const uint32_t b = __float_as_uint(f);
    const uint32_t k = b ^ ((uint32_t)((int)b >> 31) | 0x80000000u);
    return f != f ? 0u : k;
}

__device__ __forceinline__ float key_float(uint32_t k)
{
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// the two smallest of {a1 <= a2} and {b1 <= b2}
__device__ __forceinline__ void merge_low2(uint32_t& a1, uint32_t& a2, uint32_t b1, uint32_t b2)
{
    const uint32_t n2 = min(max(a1, b1), min(a2, b2));
    a1 = min(a1, b1);
    a2 = n2;
}

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ void dpp_low2(uint32_t& a1, uint32_t& a2)
{
    const uint32_t o1 = dpp_t<CTRL, ROW_MASK>(0xffffffffu, a1);
    const uint32_t o2 = dpp_t<CTRL, ROW_MASK>(0xffffffffu, a2);
    merge_low2(a1, a2, o1, o2);
}

// the two smallest of the wave's pairs, in every lane
__device__ __forceinline__ void wave_low2(uint32_t& a1, uint32_t& a2)
{
    dpp_low2<0x111>(a1, a2);
    dpp_low2<0x112>(a1, a2);
    dpp_low2<0x114>(a1, a2);
    dpp_low2<0x118>(a1, a2);
    dpp_low2<0x142, 0xA>(a1, a2);
    dpp_low2<0x143, 0xC>(a1, a2);
    a1 = lane63(a1);
    a2 = lane63(a2);
}

// The cutoff of the 4096 importances held VPT = 4096 / (64 NW) per thread
// (v: numbers >= +0 or NaN, as 1e5 * |x * probe| gives).  Wave 0 finishes
// the search after its last barrier: its threads return the cutoff and lane
// 0 stores it in L.cut; the other waves return 0 there, so a caller that
// needs the cutoff in every wave reads L.cut after a barrier.  The scratch
// may be reused after that barrier.
template <int NW>
__device__ float search_cutoff(const float (&v)[IAM_PROBES_COUNT / (64 * NW)], int quantile, SearchLds<NW>& L)
{
#pragma clang fp contract(off)
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    constexpr int VPT = IAM_PROBES_COUNT / (64 * NW);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int t = IAM_PROBES_COUNT - quantile;         // bucketMul.cl:81

    // ---- 1. keys, their range and the count of numbers
    uint32_t key[VPT];
    uint32_t kmn1 = 0xffffffffu, kmx = 0u;   // min of key - 1 (NaN keys wrap to the top), max
    int nv = 0;
#pragma unroll
    for (int k = 0; k < VPT; k++) {
        key[k] = order_key(v[k]);
        kmn1 = min(kmn1, key[k] - 1u);
        kmx = max(kmx, key[k]);
        nv += __popcll(__ballot(key[k] != 0u));
    }
    kmn1 = wave_reduce(kmn1, [](uint32_t a, uint32_t b) { return min(a, b); });
    kmx = wave_reduce(kmx, [](uint32_t a, uint32_t b) { return max(a, b); });
    if (lane == 0) {
        L.red[0][wave] = kmn1;
        L.red[1][wave] = kmx;
    }
    // the block's count: the waves' ballots summed through the histogram
    // scratch of pass 2 (cleared below before its use)
    if (lane == 0) L.H[1][0][wave] = (uint32_t)nv;
    // each wave clears its first histogram (its own region: program order
    // puts the clear before its atomics)
    reinterpret_cast<uint4*>(L.H[0][wave])[lane] = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();
    kmn1 = 0xffffffffu;
    kmx = 0u;
    nv = 0;
#pragma unroll
    for (int w = 0; w < NW; w++) {
        kmn1 = min(kmn1, L.red[0][w]);
        kmx = max(kmx, L.red[1][w]);
        nv += (int)L.H[1][0][w];
    }
    const uint32_t kmn = kmn1 + 1u;
    // bucketMul.cl:98-99: min and max from 1e30 / -1e30 (fmin / fmax skip NaN)
    const float gmin = nv ? fminf(1e30f, key_float(kmn)) : 1e30f;
    const float gmax = nv ? fmaxf(-1e30f, key_float(kmx)) : -1e30f;

    // ---- 2. radix select of the key of rank a (descending, 1-based): after
    // it, the keys whose offset from the minimum has the top bits `prefix`
    // (shift s) are the tie group of u_a: equal keys (s == 0) or one key
    const int a = min(t, nv);
    uint32_t ukey = 0u;
    int gt = 0, eq = 0;            // #(keys > ukey), #(keys == ukey)
    uint32_t a1 = 0xffffffffu, a2 = 0xffffffffu, b1 = 0xffffffffu, b2 = 0xffffffffu;
    if (a >= 1) {
        const uint32_t range = kmx - kmn;
        const int top = range ? 31 - __clz(range) : 0;
        int s = max(top - 7, 0);       // digit = (rel >> s) & (2^w - 1)
        int w = top + 1 - s;
        uint32_t prefix = 0u;          // rel >> (s + w) of the keys still in the running
        int r = a;
        int buf = 0;
        bool first = true;
        for (;;) {
            {
                uint32_t* H = L.H[buf][wave];
                const uint32_t dmask = (1u << w) - 1u;
                const int sw = first ? 0 : s + w;   // the first pass takes every number
#pragma unroll
                for (int k = 0; k < VPT; k++) {
                    const uint32_t rel = key[k] - kmn;
                    const bool in = key[k] != 0u && (first || (rel >> sw) == prefix);
                    if (in) atomicAdd(H + ((rel >> s) & dmask), 1u);
                }
            }
            __syncthreads();
            // the next pass's histogram (free: every wave has scanned it)
            reinterpret_cast<uint4*>(L.H[buf ^ 1][wave])[lane] = make_uint4(0u, 0u, 0u, 0u);
            // bins 4*lane .. 4*lane+3 summed over the waves
            int c0 = 0, c1 = 0, c2 = 0, c3 = 0;
#pragma unroll
            for (int w2 = 0; w2 < NW; w2++) {
                const uint4 h = reinterpret_cast<const uint4*>(L.H[buf][w2])[lane];
                c0 += (int)h.x;
                c1 += (int)h.y;
                c2 += (int)h.z;
                c3 += (int)h.w;
            }
            const int incl = wave_incl_sum(c0 + c1 + c2 + c3);
            const int above3 = __builtin_amdgcn_readlane(incl, 63) - incl;   // keys in bins above 4*lane+3
            const int above2 = above3 + c3, above1 = above2 + c2, above0 = above1 + c1;
            // the bin d with above(d) < r <= above(d) + count(d)
            const bool f3 = above3 < r && r <= above2, f2 = above2 < r && r <= above1;
            const bool f1 = above1 < r && r <= above0, f0 = above0 < r && r <= above0 + c0;
            const int d = 4 * lane + (f3 ? 3 : f2 ? 2 : f1 ? 1 : 0);
            const int ab = f3 ? above3 : f2 ? above2 : f1 ? above1 : above0;
            const int cd = f3 ? c3 : f2 ? c2 : f1 ? c1 : c0;
            const int src = __ffsll((long long)__ballot(f3 | f2 | f1 | f0)) - 1;
            const uint32_t dd = (uint32_t)__builtin_amdgcn_readlane(d, src);
            r -= __builtin_amdgcn_readlane(ab, src);
            const int cnt = __builtin_amdgcn_readlane(cd, src);
            prefix = (prefix << w) | dd;
            if (s == 0 || cnt == 1) {  // the bin holds cnt equal keys, or one key
                eq = cnt;
                break;
            }
            w = min(8, s);
            s -= w;
            buf ^= 1;
            first = false;
        }
        gt = a - r;                    // r is the rank left within the keys equal to ukey

        // ---- 3. the tie group's key, the two smallest keys above its bin and
        // the two largest below it (as the two smallest ~key; NaN keys, 0,
        // lie below every bin, and an absent one decodes to the NaN key,
        // which compares like -inf)
        uint32_t tmax = 0u;
#pragma unroll
        for (int k = 0; k < VPT; k++) {
            const uint32_t kb = (key[k] - kmn) >> s;
            const bool num = key[k] != 0u;
            const uint32_t da = num && kb > prefix ? key[k] : 0xffffffffu;
            const uint32_t db = num && kb >= prefix ? 0xffffffffu : ~key[k];
            tmax = max(tmax, num && kb == prefix ? key[k] : 0u);
            a2 = min(a2, max(a1, da));
            a1 = min(a1, da);
            b2 = min(b2, max(b1, db));
            b1 = min(b1, db);
        }
        wave_low2(a1, a2);
        wave_low2(b1, b2);
        tmax = wave_reduce(tmax, [](uint32_t x, uint32_t y) { return max(x, y); });
        if (lane == 0) {
            *reinterpret_cast<uint4*>(L.nb[wave]) = make_uint4(a1, a2, b1, b2);
            L.tie[wave] = tmax;
        }
        __syncthreads();
        if (wave != 0) return 0.0f;    // wave 0 finishes the search and writes the cutoff
        a1 = a2 = b1 = b2 = 0xffffffffu;
#pragma unroll
        for (int w2 = 0; w2 < NW; w2++) {
            const uint4 q = *reinterpret_cast<const uint4*>(L.nb[w2]);
            merge_low2(a1, a2, q.x, q.y);
            merge_low2(b1, b2, q.z, q.w);
            ukey = max(ukey, L.tie[w2]);
        }
        b1 = ~b1;
        b2 = ~b2;
    } else if (wave != 0) {
        return 0.0f;
    }

    // ---- 4. u_{t+o}, o = -2 .. 2, lane o + 2 computing one (ranks within two
    // of t lie within two of the tie group of u_a; ranks past the numbers
    // compare like -inf; ranks below 1 are above every bound, flagged)
    float U[5];
    {
        const int k = t + lane - 2;
        const uint32_t kk = (k > gt && k <= gt + eq) ? ukey
                          : k == gt ? a1
                          : k == gt - 1 ? a2
                          : k == gt + eq + 1 ? b1
                                             : b2;
        const float uk = k > nv ? -INFINITY : key_float(kk);
#pragma unroll
        for (int o = 0; o < 5; o++) U[o] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(uk), o));
    }
    const bool top_m1 = t - 1 < 1, top_m2 = t - 2 < 1;   // (U[0], U[1] unused then)

    // ---- 5. the reference's rounds (bucketMul.cl:139-213): one chain of
    // bounds, each round's side picked by U[2] > b (count >= target); lane r
    // keeps round r's tested bound and the decisions collect in a bit mask.
    // Round r's bracket is then rebuilt per lane: its low end is the last
    // tested bound at or before r whose count reached the target (else the
    // minimum), its high end the last one whose count did not (else the
    // maximum).
    float lo = gmin, hi = gmax;
    float b = midpoint(gmin, gmax);
    float cb = 0.0f;
    uint32_t gbits = 0u;
#pragma unroll
    for (int rd = 0; rd < 20; rd++) {
        const bool g = U[2] > b;             // count >= target: min moves
        cb = lane == rd ? b : cb;
        gbits |= (g ? 1u : 0u) << rd;
        lo = g ? b : lo;
        hi = g ? hi : b;
        b = midpoint(lo, hi);
    }
    const uint32_t upto = lane < 20 ? (2u << lane) - 1u : 0xfffffu;    // rounds 0 .. lane
    const uint32_t gl = gbits & upto, gh = ~gbits & upto;
    const float clo = gl ? __shfl(cb, 31 - __clz(gl), 64) : gmin;
    const float chi = gh ? __shfl(cb, 31 - __clz(gh), 64) : gmax;
    const bool cge = lane < 20 && ((gbits >> lane) & 1u);
    const bool cmi = gl == 0u;     // minB is still the minimum: its count is the reference's 4096 (:142)
    // lane r < 20: the stop tests of round r (bucketMul.cl:195-200)
    const bool eq_t = cge && !(U[3] > cb);                        // count == target
    const bool am1 = top_m1 || U[1] > chi, am2 = top_m2 || U[0] > chi;
    const int dmax = am1 ? 1 : am2 ? 2 : 3;                       // target - maxCount (3: 3 or more)
    const int dmin = !(U[3] > clo) ? 0 : !(U[4] > clo) ? 1 : 2;   // minCount - target (2: 2 or more)
    const bool gap_small = cmi ? (dmax <= 2 && t - dmax >= IAM_PROBES_COUNT - 2)   // 4096 - maxCount < 3
                               : dmin + dmax < 3;
    const bool stop = lane < 20 && (eq_t || __fsub_rn(chi, clo) < 0.00001f || gap_small);
    const uint64_t sm = __ballot(stop);
    // no stop: the untested midpoint after round 20 (:211-213)
    const float cut = sm ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cb), __ffsll((long long)sm) - 1)) : b;
    if (lane == 0) L.cut = cut;
    return cut;
}

}  // namespace iam
