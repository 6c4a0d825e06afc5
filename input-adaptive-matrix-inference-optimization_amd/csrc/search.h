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

// the three smallest of {a1 <= a2 <= a3} and {b1 <= b2 <= b3}: the k-th
// smallest of two sorted lists is the least max(a_i, b_j) over i + j = k
// (a_0 = b_0 below everything)
__device__ __forceinline__ void merge_low3(uint32_t& a1, uint32_t& a2, uint32_t& a3, uint32_t b1, uint32_t b2,
                                           uint32_t b3)
{
    const uint32_t n3 = min(min(a3, b3), min(max(a1, b2), max(a2, b1)));
    const uint32_t n2 = min(min(a2, b2), max(a1, b1));
    a1 = min(a1, b1);
    a2 = n2;
    a3 = n3;
}

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ void dpp_low3(uint32_t& a1, uint32_t& a2, uint32_t& a3)
{
    const uint32_t o1 = dpp_t<CTRL, ROW_MASK>(0xffffffffu, a1);
    const uint32_t o2 = dpp_t<CTRL, ROW_MASK>(0xffffffffu, a2);
    const uint32_t o3 = dpp_t<CTRL, ROW_MASK>(0xffffffffu, a3);
    merge_low3(a1, a2, a3, o1, o2, o3);
}

// the three smallest of the wave's triples, in every lane
__device__ __forceinline__ void wave_low3(uint32_t& a1, uint32_t& a2, uint32_t& a3)
{
    dpp_low3<0x111>(a1, a2, a3);
    dpp_low3<0x112>(a1, a2, a3);
    dpp_low3<0x114>(a1, a2, a3);
    dpp_low3<0x118>(a1, a2, a3);
    dpp_low3<0x142, 0xA>(a1, a2, a3);
    dpp_low3<0x143, 0xC>(a1, a2, a3);
    a1 = lane63(a1);
    a2 = lane63(a2);
    a3 = lane63(a3);
}

// The reference's rounds from U[o] = u_{t-2+o} (o = 0..4; -inf past the
// numbers; U[0], U[1] unused where t-2, t-1 < 1) and the range of the
// numbers, in every lane of the calling wave (whole waves only).
__device__ __forceinline__ float replay_rounds(const float (&U)[5], int t, float gmin, float gmax)
{
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const bool top_m1 = t - 1 < 1, top_m2 = t - 2 < 1;   // (U[0], U[1] unused then)

    // the reference's rounds (bucketMul.cl:139-213): one chain of bounds,
    // each round's side picked by U[2] > b (count >= target).  Each round's
    // bound enters lane 0 of cb while the earlier ones move up a lane
    // (whole-wave DPP shift), so after round 19 lane j holds round 19 - j's
    // bound.  (One wave runs this chain alone, so its length is its
    // instruction count: 7 per round.)
    float lo = gmin, hi = gmax;
    float b = midpoint(gmin, gmax);
    float cb = 0.0f;
#pragma unroll
    for (int rd = 0; rd < 20; rd++) {
        cb = dpp_f<0x138>(b, cb);            // wave_shr:1, lane 0 takes b
        const bool g = U[2] > b;             // count >= target: min moves
        lo = g ? b : lo;
        hi = g ? hi : b;
        b = midpoint(lo, hi);
    }
    // lane j < 20 stands for round r = 19 - j: its decision, and the bracket
    // of round r rebuilt from rounds 0 .. r (lanes j .. 19): the low end is
    // the last tested bound whose count reached the target (else the
    // minimum), the high end the last one whose count did not (else the
    // maximum)
    const bool act = lane < 20;
    const uint32_t G = (uint32_t)__ballot(act && U[2] > cb);
    const uint32_t upto = act ? 0xfffffu & ~((1u << lane) - 1u) : 0u;   // lanes j .. 19
    const uint32_t gl = G & upto, gh = ~G & upto;
    const float clo = gl ? __shfl(cb, __ffs(gl) - 1, 64) : gmin;
    const float chi = gh ? __shfl(cb, __ffs(gh) - 1, 64) : gmax;
    // (bitwise logic below: the tests are cheap and branches are not)
    const bool cge = act & (((G >> (lane & 31)) & 1u) != 0u);
    const bool cmi = gl == 0u;     // minB is still the minimum: its count is the reference's 4096 (:142)
    // the stop tests of round r (bucketMul.cl:195-200)
    const bool eq_t = cge & !(U[3] > cb);                         // count == target
    const bool am1 = top_m1 | (U[1] > chi), am2 = top_m2 | (U[0] > chi);
    const int dmax = am1 ? 1 : am2 ? 2 : 3;                       // target - maxCount (3: 3 or more)
    const int dmin = !(U[3] > clo) ? 0 : !(U[4] > clo) ? 1 : 2;   // minCount - target (2: 2 or more)
    const bool gap_min = (dmax <= 2) & (t - dmax >= IAM_PROBES_COUNT - 2);   // 4096 - maxCount < 3
    const bool gap_small = cmi ? gap_min : dmin + dmax < 3;
    const bool stop = act & (eq_t | (__fsub_rn(chi, clo) < 0.00001f) | gap_small);
    const uint64_t sm = __ballot(stop);
    // the first round that stops is the highest stopping lane; no stop: the
    // untested midpoint after round 20 (:211-213)
    return sm ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cb), 63 - __clzll((long long)sm))) : b;
}

// The cutoff of the 4096 importances held VPT = 4096 / (64 NW) per thread
// (v: numbers >= +0 or NaN, as 1e5 * |x * probe| gives).  Wave 0 finishes
// the search after its last barrier: its threads return the cutoff and lane
// 0 stores it in L.cut; the other waves return 0 there, so a caller that
// needs the cutoff in every wave reads L.cut after a barrier.  The scratch
// may be reused after that barrier.
template <int NW>
__device__ __forceinline__ float search_cutoff(const float (&v)[IAM_PROBES_COUNT / (64 * NW)], int quantile, SearchLds<NW>& L)
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
    const float cut = replay_rounds(U, t, gmin, gmax);
    if (lane == 0) L.cut = cut;
    return cut;
}


// ---------------------------------------------------------------------------
// Windowed search: the same cutoff for the walk's workgroup in three
// barriers, the serial tail done by wave 0 alone.  Importances are numbers
// >= +0 (or NaN) with the sign bit clear; their keys are their bits with
// the top bit set, so bits 30..20 of a key (the float's exponent and its
// top three mantissa bits) give 2048 coarse bins of 1/8 binade in key
// order, and a NaN's key lies above +inf's.
//   A. every thread adds its keys to the coarse histogram; each wave
//      reduces its key range (barrier);
//   B. every wave finds the coarse bins holding ranks kmin = max(1, t-2)
//      and kmax = min(n, t+2) (n numbers); the window is those bins and the
//      ones between;
//   C. a window of at most kSmallWindow keys is gathered into a list; a
//      larger one goes into 1024 fine bins, each with its count and its
//      largest and smallest key (barrier);
//   D. wave 0 ranks the list, or reads the fine bins from the top of the
//      16 that hold kmin: where kmax lies within 128 of them and no bin
//      holding a rank kmin .. kmax has more than two keys, those keys are
//      u_kmin .. u_kmax; otherwise the keys of those fine bins are gathered
//      (two more barriers) and ranked.  Either way u_{t-2} .. u_{t+2} come
//      out exactly, and wave 0 replays the reference's rounds from them
//      while the other waves run the caller's `overlap(hi)` (wave 0 runs it
//      after its tail) with hi > cutoff from the window of B (cutoff_upper),
//      so that rows certain to be selected can be listed while the search
//      finishes; a barrier then hands the cutoff to all.
// It declines (in every wave at the same step) when an importance is NaN or
// a list would be longer than kListCap; search_cutoff then finds the cutoff.  Histograms are read with one lane per NB consecutive
// bins (NB = 32 coarse, 16 fine), stored so that a wave's 16-byte reads are
// contiguous.
constexpr int kCoarseBins = 2048;
constexpr int kFineBins = 1024;
constexpr uint32_t kKeyInf = 0xff800000u;   // the window search's key of +inf (NaN keys lie above)
constexpr int kListCap = 64;
constexpr int kSmallWindow = 32;   // a window of at most this many keys is listed outright

// what wave 0 hands on after its tail: no cutoff (the radix search runs),
// a list of the fine bins' keys to gather, or the cutoff
enum : int { kWinDecline = 0, kWinList = 1, kWinDone = 3 };

template <int NW>
struct WindowLds {
    uint32_t coarse[kCoarseBins];
    uint32_t fine[kFineBins];
    uint32_t fmax[kFineBins];   // per fine bin (at its count's slot): its largest key
    uint32_t fminv[kFineBins];  // ~ its smallest key
    uint32_t list[kListCap];
    uint32_t ukey[8];           // keys of ranks t-2 .. t+2 (0: none)
    uint32_t red[2][NW];        // per wave: min key, max key
    uint32_t nlist;
    // wave 0's hand-over
    int step, nl, above;
    uint32_t rlo, rhi;
    float cut;
    float hint;                 // the hinted window's centre (thread 0 stores it before a barrier)
    // hinted pass, over the waves (LDS atomics): min key, max key, keys above
    // | keys in << 16
    uint32_t hred[3];
};

// slot of bin b in a histogram read NB bins per lane: lane l's i-th 16-byte
// read (at 1024 i + 16 l) holds bins NB l + 4i .. NB l + 4i + 3
template <int NB>
__device__ __forceinline__ int hist_slot(int b)
{
    const uint32_t u = (uint32_t)b;   // b >= 0: unsigned shifts, no rounding fix-ups of a division
    if constexpr (NB == 16)           // the same for b < 1024, as three bit fields
        return (int)(((u & 0xcu) << 6) | ((u >> 2) & 0xfcu) | (u & 3u));
    return (int)(((u >> 2) & (NB / 4 - 1)) * 256u + (u / NB) * 4u + (u & 3u));
}

__device__ __forceinline__ int coarse_bin(uint32_t key) { return (int)((key >> 20) & (kCoarseBins - 1)); }

// A key added to fine bin b < kFineBins (its count, largest and smallest
// key).  The byte offset of hist_slot<16>(b) as three bit fields: bits 0-1
// of b move to 2-3, bits 2-3 to 10-11, bits 4-9 stay.
template <int NW>
__device__ __forceinline__ void fine_add(WindowLds<NW>& W, uint32_t b, uint32_t key)
{
    const uint32_t off = (b & 0x3f0u) | ((b << 2) & 0xcu) | ((b << 8) & 0xc00u);
    atomicAdd(reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(W.fine) + off), 1u);
    atomicMax(reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(W.fmax) + off), key);
    atomicMax(reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(W.fminv) + off), ~key);
}

// The zeroing of the histograms and the list counter, by all NT threads;
// a barrier must separate it from search_window.
template <int NW>
__device__ __forceinline__ void window_clear(WindowLds<NW>& W)
{
    constexpr int NT = 64 * NW;
    constexpr int kVecs = (kCoarseBins + 3 * kFineBins) / 4;
    static_assert(offsetof(WindowLds<NW>, list) == (kCoarseBins + 3 * kFineBins) * 4, "the histograms first");
    uint4* z = reinterpret_cast<uint4*>(W.coarse);
#pragma unroll
    for (int i = 0; i < (kVecs + NT - 1) / NT; i++)
        if (i * NT + (int)threadIdx.x < kVecs) z[i * NT + threadIdx.x] = make_uint4(0u, 0u, 0u, 0u);
    if (threadIdx.x == 0) {
        W.nlist = 0u;
        W.hred[0] = 0xffffffffu;
        W.hred[1] = 0u;
        W.hred[2] = 0u;
    }
}

// One wave's scan of a histogram of 64 NB bins (keys counted in ascending
// key order): lane sums, their prefix, and the number of keys above each
// lane's bins.
template <int NB>
struct HistScan {
    int tl, abl, total;
};

template <int NB>
__device__ __forceinline__ HistScan<NB> hist_scan(const uint32_t* H)
{
    const int lane = threadIdx.x & 63;
    const uint4* H4 = reinterpret_cast<const uint4*>(H);
    uint4 h[NB / 4];
#pragma unroll
    for (int i = 0; i < NB / 4; i++) h[i] = H4[i * 64 + lane];
    int tl = 0;
#pragma unroll
    for (int i = 0; i < NB / 4; i++) tl += (int)(h[i].x + h[i].y + h[i].z + h[i].w);
    const int incl = wave_incl_sum(tl);
    const int total = __builtin_amdgcn_readlane(incl, 63);
    return HistScan<NB>{tl, total - incl, total};
}

// The bins d1 >= d2 of ranks 1 <= r1 <= r2 <= total (descending, 1-based),
// the keys above each, and d2's count.  Lanes 0..31 resolve r1 within its
// lane's NB bins, lanes 32..63 r2.
template <int NB>
__device__ __forceinline__ void hist_find2(const uint32_t* H, const HistScan<NB>& sc, int r1, int r2, int& d1,
                                           int& ab1, int& d2, int& ab2, int& c2)
{
    static_assert(NB <= 32, "a half wave per rank");
    const int lane = threadIdx.x & 63;
    const int L1 = __ffsll((long long)__ballot(sc.abl < r1 && r1 <= sc.abl + sc.tl)) - 1;
    const int L2 = __ffsll((long long)__ballot(sc.abl < r2 && r2 <= sc.abl + sc.tl)) - 1;
    const int a1 = __builtin_amdgcn_readlane(sc.abl, L1);
    const int a2 = __builtin_amdgcn_readlane(sc.abl, L2);
    const bool hf = lane >= 32;
    const int j = lane & 31;
    const int c = j < NB ? (int)H[hist_slot<NB>((hf ? L2 : L1) * NB + j)] : 0;
    const int inc = wave_incl_sum(c);
    const int above = (hf ? __builtin_amdgcn_readlane(inc, 63) : __builtin_amdgcn_readlane(inc, 31)) - inc;
    const int rb = hf ? r2 - a2 : r1 - a1;
    const uint64_t bm = __ballot(j < NB && above < rb && rb <= above + c);
    const int j1 = __ffsll((long long)(bm & 0xffffffffull)) - 1;
    const int j2 = __ffsll((long long)(bm >> 32)) + 31;
    d1 = L1 * NB + j1;
    ab1 = a1 + __builtin_amdgcn_readlane(above, j1);
    d2 = L2 * NB + (j2 - 32);
    ab2 = a2 + __builtin_amdgcn_readlane(above, j2);
    c2 = __builtin_amdgcn_readlane(c, j2);
}

// The keys of ranks t-2 .. t+2 read back from W.ukey (0: no such rank,
// which compares like -inf)
template <int NW>
__device__ __forceinline__ void read_ukeys(const WindowLds<NW>& W, float (&U)[5])
{
    const uint4 q = *reinterpret_cast<const uint4*>(W.ukey);
    const uint32_t k[5] = {q.x, q.y, q.z, q.w, W.ukey[4]};
#pragma unroll
    for (int o = 0; o < 5; o++) U[o] = k[o] ? key_float(k[o]) : -INFINITY;
}

// wave 0: u_{t-2} .. u_{t+2} from the nl listed keys: lane i's key holds
// ranks above + gt + 1 .. above + ge
template <int NW>
__device__ __forceinline__ void rank_list(WindowLds<NW>& W, int nl, int above, int t, float (&U)[5])
{
    const int lane = threadIdx.x & 63;
    const uint32_t lk = lane < nl ? W.list[lane] : 0u;
    if (lane < 5) W.ukey[lane] = 0u;
    int gt = above, ge = above;
    for (int j = 0; j < nl; j++) {
        const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)lk, j);
        gt += kj > lk ? 1 : 0;
        ge += kj >= lk ? 1 : 0;
    }
#pragma unroll
    for (int o = 0; o < 5; o++) {
        const int k = t - 2 + o;
        if (lane < nl && gt < k && k <= ge) W.ukey[o] = lk;
    }
    read_ukeys(W, U);
}

// wave 0: the reference's rounds from U, the cutoff left in W.cut
template <int NW>
__device__ __forceinline__ void window_finish(WindowLds<NW>& W, const float (&U)[5], int t, uint32_t kmn, uint32_t kmx)
{
    // bucketMul.cl:98-99: min and max from 1e30 / -1e30 (fmin / fmax skip NaN)
    const float gmin = fminf(1e30f, key_float(kmn));
    const float gmax = fmaxf(-1e30f, key_float(kmx));
    const float cut = replay_rounds(U, t, gmin, gmax);
    if ((threadIdx.x & 63) == 0) {
        W.cut = cut;
        W.step = kWinDone;
    }
}

// An upper bound of the cutoff from an upper bound `edge` > u_{t-2} (t >= 3):
// the upper edge of the coarse bin of rank kmin = t - 2, or the upper end of
// a hinted window holding that rank.  With u_j the j-th largest importance,
// gmin / gmax their range and the bracket [min, max] of the rounds, the
// reference's outcomes are (bucketMul.cl:131-213):
//   count == t            returns b with u_{t+1} <= b < u_t;
//   |maxCount-minCount|<3 returns b = the moved end: if max moved, count(b)
//                         >= minCount - 2 >= t - 2, so b < u_{t-2}; if min
//                         moved, count(b) >= t, so b < u_t;
//   max - min < 1e-5      returns an end of a bracket holding u_t (min < u_t
//                         <= max): b lies within 1e-5 (the fp32 test, so
//                         within 1.0001e-5 exactly) of u_t;
//   20 rounds             returns the midpoint of a bracket holding u_t
//                         whose width is at most (gmax - gmin) 2^-20 +
//                         ulp(gmax) (each fp32 midpoint rounds by at most
//                         half an ulp of the sum).
// With delta = max(1.0001e-5, (gmax - gmin) 2^-20 + gmax 2^-23) and
// u_t <= u_{t-2} < edge,
//   cutoff < u_{t-2} + delta < edge + delta <= hi,
// and every row whose importance reaches hi is selected.  hi is formed in
// fp32, every operation rounded to nearest (relative error at most 2^-24
// each; the scalings by powers of two are exact): the difference, the sum
// of the two terms and the sum with edge lose at most a factor
// (1 - 2^-24)^3 > 1 - 2^-22 together, 1.0002e-5f exceeds 1.0001e-5, and
// the last product by 1 + 2^-20 (itself rounded, another 1 - 2^-24) more
// than makes up for them, so hi >= edge + delta exactly.  All terms are
// >= 0 and the sum is at least 1e-5 (no denormal); an overflow gives
// +inf, which no importance reaches here (kmx is below +inf's key).  Where
// t < 3, or an importance is infinite, there is no bound: hi = NaN, which
// no importance reaches (not even +inf).
__device__ __forceinline__ float cutoff_upper(int t, float edge, uint32_t kmn, uint32_t kmx)
{
#pragma clang fp contract(off)
    if (t < 3 || kmx >= 0xff800000u) return __int_as_float(0x7fc00000);   // kmx: the key of +inf
    const float gmn = key_float(kmn), gmx = key_float(kmx);
    const float dl = fmaxf(1.0002e-5f, __fadd_rn(__fmul_rn(__fsub_rn(gmx, gmn), 0x1p-20f), __fmul_rn(gmx, 0x1p-23f)));
    return __fmul_rn(__fadd_rn(edge, dl), 1.0f + 0x1p-20f);
}

// A hint the windowed search takes: a positive normal float well inside the
// float range (the cutoff of the same matrix in the previous decode step)
__device__ __forceinline__ bool hint_usable(float h) { return h >= 1e-30f && h <= 1e30f; }

// Returns 1 with the cutoff in every wave (overlap has run in every wave,
// wave 0's with hi = NaN), 0 when declined before it ran, 2 when declined
// after it; hint_hit: the hinted window held the cutoff's ranks (in every
// wave).
//
// With a usable hint in W.hint (hinted; the same value in every wave), one pass replaces
// steps A to C: the window is [7/8 hint, 8/7 hint); each thread counts its
// keys above it and its numbers, adds the keys inside it to the fine bins,
// and a barrier sums the waves' counts and key ranges.  When the window
// holds the ranks kmin .. kmax (fewer than kmin keys above it, at least
// kmax down to its lower end), step D runs on it as on a window from B;
// otherwise the fine bins are cleared and steps A to D run.  Either way the
// keys u_{t-2} .. u_{t+2}, and so the cutoff, are the same: the hint only
// picks which window finds them.
template <int NW, typename Overlap>
__device__ __forceinline__ int search_window(const float (&v)[IAM_PROBES_COUNT / (64 * NW)], int quantile, bool hinted,
                             WindowLds<NW>& W, float& cut, bool& hint_hit, Overlap&& overlap)
{
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    constexpr int NT = 64 * NW;
    constexpr int VPT = IAM_PROBES_COUNT / NT;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int t = IAM_PROBES_COUNT - quantile;       // bucketMul.cl:81

    // The importances are >= +0 or NaN with the sign bit clear (1e5 * |x *
    // probe|), so their keys are their bits with the top bit set: one
    // instruction instead of order_key's four.  A NaN's key then lies above
    // +inf's, and the window search declines on seeing one (the radix
    // search maps NaN below every number); +0's key is not zero.
    uint32_t key[VPT];
#pragma unroll
    for (int k = 0; k < VPT; k++) key[k] = __float_as_uint(v[k]) | 0x80000000u;

    // the window of step D: its keys as a list (listed, mc keys) or in the
    // fine bins (sf: bin shift) from key base over width key units, ab_hi
    // keys above it; the ranks it holds, the key range, and the bound hi
    uint32_t kmn, kmx, base, width;
    int sf, ab_hi, kmin, kmax, mc = 0;
    bool listed = false, ready = false;
    float hi;
    float U[5];   // wave 0: u_{t-2} .. u_{t+2}
    hint_hit = false;

    // ---- E. the last rank (t = 4096, effort 1): u_{t-2} .. u_t are the
    // three smallest keys and u_{t+1}, u_{t+2} lie past the numbers.  Each
    // thread keeps its three smallest, the waves merge theirs by DPP, and
    // after one barrier every wave merges the waves' triples: wave 0 replays
    // the rounds, the others list the rows above the bound from the key just
    // above u_{t-2}.
    const bool last = t == IAM_PROBES_COUNT;
    if (last) {
        uint32_t a1 = 0xffffffffu, a2 = 0xffffffffu, a3 = 0xffffffffu, mx = 0u;
#pragma unroll
        for (int k = 0; k < VPT; k++) {
            merge_low3(a1, a2, a3, key[k], 0xffffffffu, 0xffffffffu);
            mx = max(mx, key[k]);
        }
        wave_low3(a1, a2, a3);
        mx = wave_max_u32(mx);
        if (lane == 0) {
            W.list[3 * wave] = a1;
            W.list[3 * wave + 1] = a2;
            W.list[3 * wave + 2] = a3;
            W.red[1][wave] = mx;
        }
        __syncthreads();
        kmx = W.red[1][0];
#pragma unroll
        for (int w = 1; w < NW; w++) kmx = max(kmx, W.red[1][w]);
        if (kmx > kKeyInf) return 0;   // a NaN
        uint32_t b1 = 0xffffffffu, b2 = 0xffffffffu, b3 = 0xffffffffu;
        if (lane < NW) {
            b1 = W.list[3 * lane];
            b2 = W.list[3 * lane + 1];
            b3 = W.list[3 * lane + 2];
        }
        wave_low3(b1, b2, b3);
        U[0] = key_float(b3);
        U[1] = key_float(b2);
        U[2] = key_float(b1);
        U[3] = U[4] = -INFINITY;
        kmn = b1;
        // (b3 + 1 is the key of the next float up; where b3 is +inf's key,
        // so is kmx, and there is no bound)
        hi = wave != 0 ? cutoff_upper(t, key_float(b3 + 1u), b1, kmx) : __int_as_float(0x7fc00000);
        ready = true;
    }

    // ---- H. the hinted window (hinted: the launch has a hint, uniform; its
    // value is read from LDS only then)
    const float hint = hinted ? W.hint : 0.0f;
    if (!last && hint_usable(hint)) {
        const uint32_t klo = order_key(__fmul_rn(hint, 0.875f)), khi = order_key(__fmul_rn(hint, 1.142857142857f));
        const uint32_t hw = khi - klo;
        const int hsf = hw > (uint32_t)kFineBins ? 32 - __clz(hw - 1u) - 10 : 0;
        // per thread: its keys' range, the keys above the window, and the
        // keys inside it in the high half of c_ai (at most 1024 keys a wave:
        // no carry between the halves)
        uint32_t kmn1 = 0xffffffffu, kmx1 = 0u, c_ai = 0u;
#pragma unroll
        for (int k = 0; k < VPT; k++) {
            kmn1 = min(kmn1, key[k]);
            kmx1 = max(kmx1, key[k]);
            c_ai += key[k] >= khi ? 1u : 0u;
            const uint32_t rel = key[k] - klo;
            if (rel < hw) {
                c_ai += 1u << 16;
                fine_add(W, rel >> hsf, key[k]);
            }
        }
        kmn1 = wave_min_u32(kmn1);
        kmx1 = wave_max_u32(kmx1);
        c_ai = wave_sum(c_ai);
        if (lane == 0) {
            atomicMin(&W.hred[0], kmn1);
            atomicMax(&W.hred[1], kmx1);
            atomicAdd(&W.hred[2], c_ai);   // at most 4096 keys each half: no carry between them
        }
        __syncthreads();
        kmn = W.hred[0];
        kmx = W.hred[1];
        const uint32_t cw = W.hred[2];
        const int na = (int)(cw & 0xffffu), nw = (int)(cw >> 16);
        if (kmx > kKeyInf) return 0;   // a NaN
        kmin = max(1, t - 2);
        kmax = min(IAM_PROBES_COUNT, t + 2);   // every key is a number
        if (kmin > kmax) return 0;
        if (na < kmin && na + nw >= kmax) {
            ready = true;
            hint_hit = true;
            base = klo;
            width = hw;
            sf = hsf;
            ab_hi = na;
            // (wave 0, whose tail is the search's critical path, does not
            // list rows early: it skips the bound's fp64 arithmetic)
            hi = wave != 0 ? cutoff_upper(t, key_float(khi), kmn, kmx) : __int_as_float(0x7fc00000);
        } else {   // the fine bins cleared for the full search
            uint4* z = reinterpret_cast<uint4*>(W.fine);
#pragma unroll
            for (int i = 0; i < (3 * kFineBins / 4 + NT - 1) / NT; i++)
                if (i * NT + (int)threadIdx.x < 3 * kFineBins / 4) z[i * NT + threadIdx.x] = make_uint4(0u, 0u, 0u, 0u);
            __syncthreads();
        }
    }

    if (!ready) {
        // ---- A. the coarse histogram, the waves' key ranges (a NaN's key
        // lands in a bin above +inf's, and the search declines below)
        uint32_t kmn1 = 0xffffffffu;
        kmx = 0u;
#pragma unroll
        for (int k = 0; k < VPT; k++) {
            kmn1 = min(kmn1, key[k]);
            kmx = max(kmx, key[k]);
            atomicAdd(W.coarse + hist_slot<32>(coarse_bin(key[k])), 1u);
        }
        kmn1 = wave_min_u32(kmn1);
        kmx = wave_max_u32(kmx);
        if (lane == 0) {
            W.red[0][wave] = kmn1;
            W.red[1][wave] = kmx;
        }
        __syncthreads();

        // ---- B. the window, in every wave alike
        kmn1 = 0xffffffffu;
        kmx = 0u;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            kmn1 = min(kmn1, W.red[0][w]);
            kmx = max(kmx, W.red[1][w]);
        }
        kmn = kmn1;
        if (kmx > kKeyInf) return 0;   // a NaN
        const HistScan<32> cs = hist_scan<32>(W.coarse);
        kmin = max(1, t - 2);
        kmax = min(IAM_PROBES_COUNT, t + 2);   // every key is a number
        if (kmin > kmax) return 0;
        int dhi, dlo, ab_lo, c_lo;
        hist_find2<32>(W.coarse, cs, kmin, kmax, dhi, ab_hi, dlo, ab_lo, c_lo);
        const int nc = dhi - dlo + 1;
        mc = ab_lo + c_lo - ab_hi;    // keys in the window
        base = 0x80000000u + ((uint32_t)dlo << 20);
        width = (uint32_t)nc << 20;
        sf = 10 + (nc > 1 ? 32 - __clz(nc - 1) : 0);   // 1024 fine bins cover the window
        listed = mc <= kSmallWindow;

        // ---- C. the window's list or its fine histogram
        if (listed) {
#pragma unroll
            for (int k = 0; k < VPT; k++)
                if (key[k] - base < width) W.list[atomicAdd(&W.nlist, 1u)] = key[k];
        } else {
#pragma unroll
            for (int k = 0; k < VPT; k++) {
                const uint32_t rel = key[k] - base;
                if (rel < width) fine_add(W, rel >> sf, key[k]);
            }
        }
        __syncthreads();
        hi = wave != 0 ? cutoff_upper(t, __uint_as_float((uint32_t)(dhi + 1) << 20), kmn, kmx)
                       : __int_as_float(0x7fc00000);
    }

    // ---- D. wave 0: u_{t-2} .. u_{t+2} (E has them) and the rounds
    if (wave == 0) {
        bool rounds = true;
        if (last) {
        } else if (listed) {
            rank_list(W, mc, ab_hi, t, U);
        } else {
            // the fine bins of window ranks r1 = kmin - ab_hi .. r2 = kmax - ab_hi:
            // from the top bin of the lane whose 16 bins hold r1, lane l reads
            // bins top - 2l and top - 2l - 1.  Where r2 lies within those 128
            // bins and no bin holding a rank r1 .. r2 has more than two keys,
            // their largest and smallest keys are u_kmin .. u_kmax.
            const HistScan<16> fs = hist_scan<16>(W.fine);
            const int r1 = kmin - ab_hi, r2 = kmax - ab_hi;
            const int L1 = __ffsll((long long)__ballot(fs.abl < r1 && r1 <= fs.abl + fs.tl)) - 1;
            const int top = 16 * L1 + 15;
            const int a1 = __builtin_amdgcn_readlane(fs.abl, L1);    // window keys above bin top
            const int f0 = top - 2 * lane, f1 = f0 - 1;
            const int s0 = hist_slot<16>(max(f0, 0)), s1 = hist_slot<16>(max(f1, 0));
            const int c0 = f0 >= 0 ? (int)W.fine[s0] : 0, c1 = f1 >= 0 ? (int)W.fine[s1] : 0;
            const uint32_t x0 = W.fmax[s0], n0 = ~W.fminv[s0], x1 = W.fmax[s1], n1 = ~W.fminv[s1];
            const int incl = wave_incl_sum(c0 + c1);
            const int e0 = a1 + incl - c0 - c1, e1 = e0 + c0;      // window keys above bins f0, f1
            const bool ov0 = c0 > 0 && e0 < r2 && e0 + c0 >= r1, ov1 = c1 > 0 && e1 < r2 && e1 + c1 >= r1;
            const bool direct = __ballot((ov0 && c0 > 2) || (ov1 && c1 > 2)) == 0ull &&
                                a1 + __builtin_amdgcn_readlane(incl, 63) >= r2;
            if (direct) {
                // each lane's keys go to the slots of their ranks: e0 + 1 (x0),
                // e0 + 2 (n0), e1 + 1 (x1), e1 + 2 (n1), counted from t - 2
                if (lane < 5) W.ukey[lane] = 0u;
                const int o0 = ab_hi + e0 + 1 - (t - 2), o1 = ab_hi + e1 + 1 - (t - 2);
                if (c0 >= 1 && (unsigned)o0 < 5u) W.ukey[o0] = x0;
                if (c0 == 2 && (unsigned)(o0 + 1) < 5u) W.ukey[o0 + 1] = n0;
                if (c1 >= 1 && (unsigned)o1 < 5u) W.ukey[o1] = x1;
                if (c1 == 2 && (unsigned)(o1 + 1) < 5u) W.ukey[o1 + 1] = n1;
                read_ukeys(W, U);
            } else {   // list the keys of the fine bins flo .. fhi
                rounds = false;
                int fhi, ab_f, flo, ab_flo, c_flo;
                hist_find2<16>(W.fine, fs, r1, r2, fhi, ab_f, flo, ab_flo, c_flo);
                if (lane == 0) {
                    const int nl = ab_flo + c_flo - ab_f;
                    W.step = nl > kListCap ? kWinDecline : kWinList;
                    W.nl = nl;
                    W.above = ab_hi + ab_f;
                    W.rlo = (uint32_t)flo << sf;
                    W.rhi = min((uint32_t)(fhi + 1) << sf, width);
                }
            }
        }
        if (rounds) window_finish(W, U, t, kmn, kmx);
    }
    overlap(hi);
    __syncthreads();
    const int step2 = W.step;
    if (step2 == kWinDone) {
        cut = W.cut;
        return 1;
    }
    if (step2 == kWinDecline) return 2;
    // the fine bins' keys, gathered (the list counter is still zero: the
    // window was not listed)
    {
        const uint32_t rlo = W.rlo, rhi = W.rhi;
#pragma unroll
        for (int k = 0; k < VPT; k++) {
            const uint32_t rel = key[k] - base;
            if (rel >= rlo && rel < rhi) W.list[atomicAdd(&W.nlist, 1u)] = key[k];
        }
    }
    __syncthreads();
    if (wave == 0) {
        float U[5];
        rank_list(W, W.nl, W.above, t, U);
        window_finish(W, U, t, kmn, kmx);
    }
    __syncthreads();
    cut = W.cut;
    return 1;
}

}  // namespace iam
