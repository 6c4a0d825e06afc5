/*
 * CPU oracle for the input-adaptive sparse decode path (see oracle.h).
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/, by __graft_entry__.smoke() as
 * the checker and by bench.py's cpu_baseline leg.  The product library never
 * links or calls it.  Built with -O2 -ffp-contract=off -fno-fast-math so every
 * fp32 operation is a single IEEE-rounded operation.
 *
 * How each function is pinned (tests/test_oracle.py, against the fixtures in
 * tests/golden/):
 *   orc_f32_to_f16 / orc_f16_to_f32 /
 *   orc_f64_to_f16 ..................... numpy astype(float16/float32) on 2^20
 *                                        values incl. subnormals, inf, ties
 *   orc_pack_fp16 / orc_unpack_fp16 .... the 5 verify_packing cases
 *                                        (preprocess_layer_fixed_gpu.py:340-346)
 *   orc_bucketize ...................... fixtures written by importing the
 *                                        reference bucketize_fp16_packed
 *                                        (tests/golden/make_fixtures.py) plus
 *                                        structural invariants
 *   orc_np_pairwise_sum_f32 ............ np.add.reduce on float32 rows
 *   orc_effort_quantile ................ KAT {1.0:0, 0.5:2047, 0.25:3071, ...}
 *   orc_find_cutoff .................... hand-traced known answers on dyadic
 *                                        inputs, closed-form special cases
 *                                        (x = 0, constant, two-level), bracket
 *                                        invariants on random inputs, and the
 *                                        reference's own CPU restatement of the
 *                                        importance (test_cutoff_binary_search.cpp:223-237)
 *   orc_select_rows .................... brute force over rows, channel-3 only
 *   orc_bucket_walk .................... all rows selected == dense GEMV with
 *                                        the packed matrix (numpy float64);
 *                                        one-hot x; x = 0
 *   orc_rmsnorm_gain, orc_silu_mul,
 *   orc_rope, orc_attention_f16kv ...... textbook numpy float64 forms
 *   orc_attention_f32rep ............... one position (output = that V row
 *                                        exactly), equal keys (the mean of V),
 *                                        the textbook float64 form, dyadic
 *                                        scores (exact tree sums), and the
 *                                        overflow to NaN above 88.72
 *   orc_rope_kv_rep32 .................. orc_rope + an index-wise repeat
 *   orc_matmul_f16_dense ............... numpy float64 GEMV, exact sums on
 *                                        dyadic inputs, one-hot x (a column
 *                                        copy), and a reordering that a
 *                                        wrong tree gives
 *   orc_rope_table ..................... numpy float32 cos/sin of the same
 *                                        angles (within 1 ulp)
 *   orc_argmax ......................... numpy argmax (first maximum)
 *   orc_layer_forward,
 *   orc_model_forward .................. composition of the above; checked
 *                                        step by step against a re-composition
 *                                        from the separately pinned primitives
 *                                        (op order, gains, residuals, KV slot)
 *                                        on a 1-layer model over 3 positions
 */
#include "oracle.h"

#include <math.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* fp16                                                                       */
/* ------------------------------------------------------------------------- */

float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            /* subnormal: mant * 2^-24, normalise */
            int e = -1;
            do {
                e++;
                mant <<= 1;
            } while ((mant & 0x400u) == 0);
            mant &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                        /* inf / nan */
        if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
    if (ax >= 0x38800000u) {                        /* normal fp16 */
        uint32_t e = (ax >> 23) - 127 + 15;
        uint32_t mant = ax & 0x7fffffu;
        uint32_t h = (e << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (ax < 0x33000000u) return (uint16_t)sign;   /* < 2^-25: to zero (tie to even) */
    {                                               /* subnormal fp16 */
        int e = (int)(ax >> 23) - 127;              /* -25 .. -15 */
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;  /* value = m * 2^(e-23) */
        int shift = -(e + 1);                       /* n = m * 2^(e+1) */
        uint32_t n = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (n & 1u))) n++;
        return (uint16_t)(sign | n);
    }
}

uint16_t orc_f64_to_f16(double d)
{
    uint64_t x;
    memcpy(&x, &d, 8);
    uint16_t sign = (uint16_t)((x >> 48) & 0x8000u);
    uint64_t ax = x & 0x7fffffffffffffffULL;
    if (ax >= 0x7ff0000000000000ULL) {                 /* inf / nan */
        if (ax == 0x7ff0000000000000ULL) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | ((ax >> 42) & 0x3ffu));
    }
    int e = (int)(ax >> 52) - 1023;
    uint64_t m = ax & 0xfffffffffffffULL;
    if (e >= 16) return (uint16_t)(sign | 0x7c00u);
    if (e >= -14) {                                    /* normal fp16 */
        uint32_t h = ((uint32_t)(e + 15) << 10) | (uint32_t)(m >> 42);
        uint64_t rem = m & ((1ULL << 42) - 1), half = 1ULL << 41;
        if (rem > half || (rem == half && (h & 1u))) h++;  /* a carry may give inf */
        return (uint16_t)(sign | h);
    }
    if (e < -25) return sign;                          /* below 2^-25: to zero */
    {                                                  /* subnormal fp16 */
        uint64_t mm = m | (1ULL << 52);                /* value = mm * 2^(e-52) */
        int shift = 28 - e;                            /* n = value * 2^24 */
        uint64_t n = mm >> shift;
        uint64_t rem = mm & ((1ULL << shift) - 1), half = 1ULL << (shift - 1);
        if (rem > half || (rem == half && (n & 1u))) n++;
        return (uint16_t)(sign | n);
    }
}

void orc_f64_to_f16_n(const double* in, uint16_t* out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = orc_f64_to_f16(in[i]);
}

void orc_f32_to_f16_n(const float* in, uint16_t* out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(in[i]);
}

void orc_f16_to_f32_n(const uint16_t* in, float* out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(in[i]);
}

/* preprocess_layer_fixed_gpu.py:40-66 */
uint16_t orc_pack_fp16(float value, int position)
{
    uint16_t bits = orc_f32_to_f16(value);
    return (uint16_t)((bits & 0xFFF0u) | ((unsigned)position & 0xFu));
}

/* preprocess_layer_fixed_gpu.py:69-89 */
void orc_unpack_fp16(uint16_t packed, float* value, int* position)
{
    *position = packed & 0xF;
    *value = orc_f16_to_f32((uint16_t)(packed & 0xFFF0u));
}

/* ------------------------------------------------------------------------- */
/* synthetic data                                                             */
/* ------------------------------------------------------------------------- */

#define GOLDEN 0x9E3779B97F4A7C15ULL

static uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

static uint64_t stream_key(uint64_t seed, uint64_t tensor_id)
{
    return mix64(mix64(seed + GOLDEN) ^ (tensor_id * 0xD1B54A32D192ED03ULL));
}

double orc_gen_normal(uint64_t seed, uint64_t tensor_id, uint64_t n)
{
    uint64_t key = stream_key(seed, tensor_id);
    uint64_t s = 0;
    for (int j = 0; j < 6; j++) {
        uint64_t u = mix64(key + (n * 6 + (uint64_t)j + 1) * GOLDEN);
        s += (u & 0xffffffffULL) + (u >> 32);
    }
    int64_t c = (int64_t)s - (int64_t)(6ULL << 32);
    return (double)c * (1.0 / 4294967296.0);
}

uint32_t orc_gen_u32(uint64_t seed, uint64_t tensor_id, uint64_t n)
{
    uint64_t key = stream_key(seed, tensor_id);
    return (uint32_t)(mix64(key + (n + 1) * GOLDEN) & 0xffffffffULL);
}

void orc_gen_f16(uint64_t seed, uint64_t tensor_id, size_t count, double mean, double sigma,
                 uint16_t* out)
{
    for (size_t i = 0; i < count; i++) {
        double v = mean + sigma * orc_gen_normal(seed, tensor_id, i);
        out[i] = orc_f64_to_f16(v);
    }
}

void orc_gen_f32(uint64_t seed, uint64_t tensor_id, size_t count, double mean, double sigma,
                 float* out)
{
    for (size_t i = 0; i < count; i++) {
        double v = mean + sigma * orc_gen_normal(seed, tensor_id, i);
        out[i] = (float)v;
    }
}

void orc_gen_tokens(uint64_t seed, uint64_t tensor_id, size_t count, uint32_t vocab, int32_t* out)
{
    for (size_t i = 0; i < count; i++) {
        uint64_t u = orc_gen_u32(seed, tensor_id, i);
        out[i] = (int32_t)((u * (uint64_t)vocab) >> 32);
    }
}

/* ------------------------------------------------------------------------- */
/* bucket layout producer                                                     */
/* ------------------------------------------------------------------------- */

/* numpy's float32 pairwise summation (loops_utils.h.src, PW_BLOCKSIZE 128),
 * which np.mean applies along a contiguous reduction axis. */
float orc_np_pairwise_sum_f32(const float* a, ptrdiff_t n)
{
    if (n < 8) {
        float res = -0.0f;
        for (ptrdiff_t i = 0; i < n; i++) res += a[i];
        return res;
    } else if (n <= 128) {
        float r[8];
        ptrdiff_t i;
        for (int j = 0; j < 8; j++) r[j] = a[j];
        for (i = 8; i < n - (n % 8); i += 8) {
            for (int j = 0; j < 8; j++) r[j] += a[i + j];
        }
        float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        for (; i < n; i++) res += a[i];
        return res;
    } else {
        ptrdiff_t n2 = n / 2;
        n2 -= n2 % 8;
        return orc_np_pairwise_sum_f32(a, n2) + orc_np_pairwise_sum_f32(a + n2, n - n2);
    }
}

/* bucketize_fp16_packed, preprocess_layer_fixed_gpu.py:110-242.
 *   probes  :145, :154   fp16(mean_j |W[j,i]|), float32 sum in j order
 *   sort    :163-174     |w| descending within each bucket of 16; equal
 *                        magnitudes keep their original order
 *   layout  :182-188     row = i*16 + rank, column = bucket
 *   packing :192-200     (fp16 bits & 0xFFF0) | position
 *   stats   :211-221     fp16(mean_b |sorted value|) in all 4 channels */
int orc_bucketize(const uint16_t* W, int out_dim, int in_dim,
                  uint16_t* buckets, uint16_t* stats, uint16_t* probes)
{
    if (out_dim % 16 != 0 || out_dim <= 0 || in_dim <= 0) return -1;
    const int nb = out_dim / 16;
    const size_t R = (size_t)in_dim * 16;

    /* probes: reduction over the non-contiguous axis of the F-ordered W.T, so
     * numpy adds whole columns in order: acc += |W[j, :]| for j = 0.. */
    float* acc = (float*)calloc((size_t)in_dim, sizeof(float));
    for (int j = 0; j < out_dim; j++) {
        const uint16_t* row = W + (size_t)j * in_dim;
        for (int i = 0; i < in_dim; i++) acc[i] = acc[i] + fabsf(orc_f16_to_f32(row[i]));
    }
    for (int i = 0; i < in_dim; i++) probes[i] = orc_f32_to_f16(acc[i] / (float)out_dim);
    free(acc);

    float* absrow = (float*)malloc((size_t)nb * 16 * sizeof(float)); /* [rank][bucket] */
    for (int i = 0; i < in_dim; i++) {
        for (int b = 0; b < nb; b++) {
            uint16_t v[16];
            float key[16];
            int idx[16];
            for (int p = 0; p < 16; p++) {
                v[p] = W[(size_t)(b * 16 + p) * in_dim + i];
                key[p] = fabsf(orc_f16_to_f32(v[p]));
                idx[p] = p;
            }
            /* stable insertion sort, descending */
            for (int a = 1; a < 16; a++) {
                int t = idx[a];
                int c = a - 1;
                while (c >= 0 && key[idx[c]] < key[t]) {
                    idx[c + 1] = idx[c];
                    c--;
                }
                idx[c + 1] = t;
            }
            for (int k = 0; k < 16; k++) {
                int p = idx[k];
                size_t r = (size_t)i * 16 + (size_t)k;
                buckets[r * nb + b] = (uint16_t)((v[p] & 0xFFF0u) | (unsigned)p);
                absrow[(size_t)k * nb + b] = key[p];
            }
        }
        for (int k = 0; k < 16; k++) {
            size_t r = (size_t)i * 16 + (size_t)k;
            float s = 0.0f + orc_np_pairwise_sum_f32(absrow + (size_t)k * nb, nb);
            uint16_t m = orc_f32_to_f16(s / (float)nb);
            stats[r * 4 + 0] = m;
            stats[r * 4 + 1] = m;
            stats[r * 4 + 2] = m;
            stats[r * 4 + 3] = m;
        }
    }
    free(absrow);
    (void)R;
    return 0;
}

/* ------------------------------------------------------------------------- */
/* cutoff                                                                     */
/* ------------------------------------------------------------------------- */

/* bucket_mul.hpp:164 (effort is a float, widened to double) */
int orc_effort_quantile(float effort)
{
    return (int)((double)(ORC_PROBES_COUNT - 1) * (1.0 - (double)effort));
}

/* bucketMul.cl:101-117 */
void orc_importance(const float* x, const uint16_t* probes, int exp_no, float* imp)
{
    const uint16_t* p = probes + (size_t)exp_no * ORC_PROBES_COUNT;
    for (int i = 0; i < ORC_PROBES_COUNT; i++) {
        float pv = orc_f16_to_f32(p[i]);
        float prod = x[i] * pv;
        imp[i] = ORC_CUTOFF_SCALE * fabsf(prod);
    }
}

/* bucketMul.cl:119-213; the whole-workgroup min/max/count reductions are
 * order-free, which is what the LDS-tree twin at :221-345 computes. */
float orc_find_cutoff_imp(const float* imp, int quantile, orc_cutoff_trace* tr)
{
    const int target = ORC_PROBES_COUNT - quantile;          /* :81 */
    float gmin = 1e30f, gmax = -1e30f;                         /* :98-99 */
    for (int i = 0; i < ORC_PROBES_COUNT; i++) {
        gmin = fminf(gmin, imp[i]);
        gmax = fmaxf(gmax, imp[i]);
    }
    float minB = gmin, maxB = gmax;
    float bound = (gmin + gmax) / 2.0f;                        /* :139 */
    int minC = ORC_PROBES_COUNT, maxC = 0;                     /* :142-143 */
    if (tr) {
        memset(tr, 0, sizeof(*tr));
        tr->init_min = gmin;
        tr->init_max = gmax;
    }
    for (int loop = 0; loop < ORC_MAX_ROUNDS; loop++) {        /* :148 */
        int count = 0;
        for (int i = 0; i < ORC_PROBES_COUNT; i++) count += (imp[i] > bound) ? 1 : 0; /* :155 */
        if (count < target) {                                  /* :178-186 */
            maxB = bound;
            maxC = count;
        } else {
            minB = bound;
            minC = count;
        }
        float next = (minB + maxB) / 2.0f;                     /* :190 */
        if (tr) {
            tr->rounds = loop + 1;
            tr->bounds[loop] = bound;
            tr->counts[loop] = count;
            tr->final_min = minB;
            tr->final_max = maxB;
            tr->final_min_count = minC;
            tr->final_max_count = maxC;
        }
        int gap = maxC - minC;
        if (gap < 0) gap = -gap;
        if (count == target || (maxB - minB < 0.00001f) || gap < 3) { /* :195-200 */
            if (tr) tr->converged = 1;
            return bound;
        }
        bound = next;
    }
    return bound;                                              /* :211-213 */
}

float orc_find_cutoff(const float* x, const uint16_t* probes, int exp_no, int quantile,
                      orc_cutoff_trace* tr)
{
    float imp[ORC_PROBES_COUNT];
    orc_importance(x, probes, exp_no, imp);
    return orc_find_cutoff_imp(imp, quantile, tr);
}

/* ------------------------------------------------------------------------- */
/* selection and walk                                                         */
/* ------------------------------------------------------------------------- */

/* prepareDispatch, bucketMul.cl:362-385 (stats indexed with the reference's
 * fixed 4-channel stride; the stats_channels argument must be 4 to match). */
int64_t orc_select_rows(const float* x, const uint16_t* stats, int stats_channels,
                        int exp_no, int expert_rows, int in_size, float cutoff,
                        uint8_t* mask)
{
    int64_t s = 0;
    const size_t off = (size_t)expert_rows * (size_t)exp_no;
    #pragma omp parallel for schedule(static) reduction(+ : s)
    for (int r = 0; r < expert_rows; r++) {
        size_t gi = off + (size_t)r;
        float avg = orc_f16_to_f32(stats[gi * (size_t)stats_channels + 3]);
        int input = r / 16;
        uint8_t sel = 0;
        if (input < in_size) {
            float val = x[input];
            float prod = val * avg;
            float imp = ORC_CUTOFF_SCALE * fabsf(prod);
            sel = (imp >= cutoff) ? 1 : 0;
        }
        mask[r] = sel;
        s += sel;
    }
    return s;
}

/* Block-structured selection (THESIS p.42-43, future work; not in the
 * reference's code): the inputs 0.. are taken in blocks of `block`
 * consecutive ones, and row 16*i + k (i < in_size) is selected when row
 * 16*u + k passes the per-row test of orc_select_rows for some input u of
 * i's block (u < in_size); rows of inputs past in_size stay unselected, as
 * in the per-row test.  block = 1 is orc_select_rows. */
int64_t orc_select_rows_block(const float* x, const uint16_t* stats, int stats_channels,
                              int exp_no, int expert_rows, int in_size, float cutoff, int block,
                              uint8_t* mask)
{
    int64_t s = orc_select_rows(x, stats, stats_channels, exp_no, expert_rows, in_size, cutoff, mask);
    if (block <= 1) return s;
    const int inputs = (expert_rows + 15) / 16;
    uint8_t* blk = (uint8_t*)calloc((size_t)((inputs + block - 1) / block) * 16, 1);
    for (int r = 0; r < expert_rows; r++)
        if (mask[r]) blk[(size_t)(r / 16 / block) * 16 + (r % 16)] = 1;
    s = 0;
    for (int r = 0; r < expert_rows; r++) {
        mask[r] = r / 16 < in_size ? blk[(size_t)(r / 16 / block) * 16 + (r % 16)] : 0;   /* past in_size: skipped */
        s += mask[r];
    }
    free(blk);
    return s;
}

/* bucketMul (bucketMul.cl:392-447) + bucketIntegrate (:453-497): every
 * selected row contributes x*packed_w at output col*16 + (bits & 15). */
void orc_bucket_walk(const uint16_t* buckets, int bucket_cols, int exp_no, int expert_rows,
                     const uint8_t* mask, const float* x, float* y, int acc64)
{
    const int C = bucket_cols;
    const int m = C * 16;
    const size_t off = (size_t)expert_rows * (size_t)exp_no;
    /* threads own column ranges (the outputs c*16 .. c*16+15 of column c
     * only receive weights of column c) and each walks the rows in
     * ascending order, so every output is summed in the same order as with
     * one thread */
    const int CB = 16;
    const int nblk = (C + CB - 1) / CB;
    if (acc64) {
        double* acc = (double*)calloc((size_t)m, sizeof(double));
        #pragma omp parallel for schedule(static)
        for (int cb = 0; cb < nblk; cb++) {
            const int c0 = cb * CB, c1 = c0 + CB < C ? c0 + CB : C;
            for (int r = 0; r < expert_rows; r++) {
                if (!mask[r]) continue;
                double xv = (double)x[r / 16];
                const uint16_t* w = buckets + (off + (size_t)r) * (size_t)C;
                for (int c = c0; c < c1; c++) {
                    acc[c * 16 + (w[c] & 15)] += xv * (double)orc_f16_to_f32(w[c]);
                }
            }
        }
        for (int o = 0; o < m; o++) y[o] = (float)acc[o];
        free(acc);
    } else {
        for (int o = 0; o < m; o++) y[o] = 0.0f;
        #pragma omp parallel for schedule(static)
        for (int cb = 0; cb < nblk; cb++) {
            const int c0 = cb * CB, c1 = c0 + CB < C ? c0 + CB : C;
            for (int r = 0; r < expert_rows; r++) {
                if (!mask[r]) continue;
                float xv = x[r / 16];
                const uint16_t* w = buckets + (off + (size_t)r) * (size_t)C;
                for (int c = c0; c < c1; c++) {
                    float prod = xv * orc_f16_to_f32(w[c]);
                    y[c * 16 + (w[c] & 15)] += prod;
                }
            }
        }
    }
}

/* the selection used by orc_bucketmul (and so by the layer and model
 * forwards): blocks of g_sel_block inputs for efforts below g_sel_below */
static int g_sel_block = 1;
static float g_sel_below = 2.0f;

void orc_set_selection_block(int block, float below_effort)
{
    g_sel_block = block > 1 ? block : 1;
    g_sel_below = below_effort;
}

int64_t orc_bucketmul(const float* x, const uint16_t* stats, const uint16_t* probes,
                      const uint16_t* buckets, int exp_no, int in_size, int bucket_cols,
                      int expert_rows, float effort, float* y, float* cutoff_out,
                      uint8_t* mask_out, int acc64)
{
    int q = orc_effort_quantile(effort);
    float cutoff = orc_find_cutoff(x, probes, exp_no, q, NULL);
    uint8_t* mask = mask_out ? mask_out : (uint8_t*)malloc((size_t)expert_rows);
    const int blk = g_sel_block > 1 && effort < g_sel_below ? g_sel_block : 1;
    int64_t s = orc_select_rows_block(x, stats, 4, exp_no, expert_rows, in_size, cutoff, blk, mask);
    orc_bucket_walk(buckets, bucket_cols, exp_no, expert_rows, mask, x, y, acc64);
    if (cutoff_out) *cutoff_out = cutoff;
    if (!mask_out) free(mask);
    return s;
}

/* ------------------------------------------------------------------------- */
/* layer kernels                                                              */
/* ------------------------------------------------------------------------- */

/* rmsNorm32fast (aux.cl:156-196): 256 partial sums of n/256 consecutive
 * squares, a 256-way tree, scale = 1/sqrt(sum/n + eps); then mul16x32
 * (aux.cl:434-440) by the fp16 gain.  The reference's rsqrt is the fast-math
 * approximation; here it is the exactly rounded value. */
void orc_rmsnorm_gain(const float* in, const uint16_t* gain, int n, float eps, float* out)
{
    float part[256];
    if (n % 256 == 0) {
        int per = n / 256;
        for (int t = 0; t < 256; t++) {
            float s = 0.0f;
            for (int i = t * per; i < (t + 1) * per; i++) {
                float sq = in[i] * in[i];
                s += sq;
            }
            part[t] = s;
        }
        for (int s = 128; s > 0; s >>= 1)
            for (int t = 0; t < s; t++) part[t] += part[t + s];
    } else {
        float s = 0.0f;
        for (int i = 0; i < n; i++) {
            float sq = in[i] * in[i];
            s += sq;
        }
        part[0] = s;
    }
    float mean = part[0] / (float)n;
    float scale = (float)(1.0 / sqrt((double)(mean + eps)));
    for (int i = 0; i < n; i++) {
        float v = in[i] * scale;
        out[i] = orc_f16_to_f32(gain[i]) * v;
    }
}

/* matrix.cl:27-32 */
void orc_silu_mul(const float* x1, const float* x3, int n, float* out)
{
    for (int i = 0; i < n; i++) {
        double g = (double)x1[i];
        out[i] = (float)((double)x3[i] * g / (1.0 + exp(-g)));
    }
}

/* attention.hpp:207-226 */
void orc_rope_table(double theta, int head_dim, int max_pos, float* table)
{
    int half = head_dim / 2;
    for (int pos = 0; pos < max_pos; pos++) {
        for (int i = 0; i < half; i++) {
            double exponent = (2.0 * i) / head_dim;
            float freq = (float)(1.0f / pow(theta, exponent));
            float angle = (float)pos * freq;
            table[((size_t)pos * half + i) * 2 + 0] = cosf(angle);
            table[((size_t)pos * half + i) * 2 + 1] = sinf(angle);
        }
    }
}

/* rope_mx, aux.cl:227-248 (rotate-half pairs d, d + head_dim/2) */
void orc_rope(const float* in, const float* table_row, int n_heads, int head_dim, float* out)
{
    int half = head_dim / 2;
    for (int h = 0; h < n_heads; h++) {
        const float* m = in + (size_t)h * head_dim;
        float* o = out + (size_t)h * head_dim;
        for (int d = 0; d < head_dim; d++) {
            int fi = d % half;
            float c = table_row[fi * 2], s = table_row[fi * 2 + 1];
            if (d < half) {
                float a = m[d] * c, b = m[d + half] * s;
                o[d] = a - b;
            } else {
                float a = m[d] * c, b = m[d - half] * s;
                o[d] = a + b;
            }
        }
    }
}

/* aux.cl:442-452 */
void orc_embed(const uint16_t* table, int cols, int token, float* out)
{
    for (int i = 0; i < cols; i++) out[i] = orc_f16_to_f32(table[(size_t)token * cols + i]);
}

/* bucketMul.cl:517-520 */
void orc_add(const float* a, const float* b, int n, float* out)
{
    for (int i = 0; i < n; i++) out[i] = a[i] + b[i];
}

/* dotSetScore2 (aux.cl:497-540): s = q.k / sqrt(hd); sum_of_exps32_mx +
 * softmax_add32_mx (aux.cl:204-225): p = exp(s)/sum exp(s); sumScores32
 * (aux.cl:370-384): o = sum_t p v_t.  Query head h reads KV head
 * h / (n_heads/n_kv) (repeat4x32, aux.cl:266-275).  Evaluated in fp64 with
 * no maximum subtracted before exp, as the reference does (so a score above
 * log(DBL_MAX) ~ 709.78 overflows to inf and the head's outputs are NaN). */
void orc_attention_f16kv(const float* q, const uint16_t* kcache, const uint16_t* vcache,
                         int n_tok, int n_heads, int n_kv, int head_dim, float* out)
{
    int rep = n_heads / n_kv;
    double inv = 1.0 / sqrt((double)head_dim);
    /* heads are independent: one per thread at a time */
    #pragma omp parallel for schedule(static)
    for (int h = 0; h < n_heads; h++) {
        double* sc = (double*)malloc(sizeof(double) * (size_t)(n_tok > 0 ? n_tok : 1));
        int kv = h / rep;
        const float* qh = q + (size_t)h * head_dim;
        for (int t = 0; t < n_tok; t++) {
            const uint16_t* k = kcache + ((size_t)t * n_kv + kv) * head_dim;
            double d = 0.0;
            for (int j = 0; j < head_dim; j++) d += (double)qh[j] * (double)orc_f16_to_f32(k[j]);
            sc[t] = d * inv;
        }
        double den = 0.0;
        for (int t = 0; t < n_tok; t++) {
            sc[t] = exp(sc[t]);
            den += sc[t];
        }
        for (int j = 0; j < head_dim; j++) {
            double acc = 0.0;
            for (int t = 0; t < n_tok; t++) {
                const uint16_t* v = vcache + ((size_t)t * n_kv + kv) * head_dim;
                acc += sc[t] * (double)orc_f16_to_f32(v[j]);
            }
            out[(size_t)h * head_dim + j] = (float)(acc / den);
        }
        free(sc);
    }
}

/* The reference's own attention path in fp32 over its cache layout: K and V
 * repeated to every query head, [ctx][n_heads][head_dim] fp32 per layer
 * (model.hpp:97-98, attention.hpp:281-309).
 *   dotSetScore2 (aux.cl:497-540): the head_dim products q[d]*k[d] summed by
 *     the work-group tree (stride head_dim/2 down to 1: p[i] += p[i+stride]),
 *     then divided by sqrt((float)head_dim);
 *   sum_of_exps32_mx (aux.cl:204-210): e_t = exp(s_t), no maximum
 *     subtracted; the reference adds them with float atomics in whatever
 *     order the work-items run.  Here the order is fixed: the positions in
 *     splits of ORC_ATT32_SPLIT, each split summed in position order, then
 *     the splits in order;
 *   softmax_add32_mx (aux.cl:219-225): p_t = exp(s_t) / sum;
 *   sumScores32 (aux.cl:370-384): o[d] = sum_t p_t * v_t[d] in fp32; the
 *     reference runs one sequential loop, here each split's products are
 *     summed in position order and the splits' sums added in split order.
 * Every operation is one IEEE fp32 operation (no contraction); expf is the C
 * library's.  A score above log(FLT_MAX) ~ 88.72 makes e_t inf and the
 * head's outputs NaN, as in the reference. */
void orc_attention_f32rep(const float* q, const float* kcache, const float* vcache, int n_tok,
                          int n_heads, int head_dim, float* out)
{
    const float root = sqrtf((float)head_dim);
    const int nsplit = (n_tok + ORC_ATT32_SPLIT - 1) / ORC_ATT32_SPLIT;
    #pragma omp parallel for schedule(static)
    for (int h = 0; h < n_heads; h++) {
        float* e = (float*)malloc(sizeof(float) * (size_t)(n_tok > 0 ? n_tok : 1));
        float* lp = (float*)malloc(sizeof(float) * (size_t)head_dim);
        const float* qh = q + (size_t)h * head_dim;
        for (int t = 0; t < n_tok; t++) {
            const float* k = kcache + ((size_t)t * n_heads + h) * head_dim;
            for (int d = 0; d < head_dim; d++) lp[d] = qh[d] * k[d];
            for (int st = head_dim / 2; st > 0; st >>= 1)
                for (int i = 0; i < st; i++) lp[i] = lp[i] + lp[i + st];
            e[t] = expf(lp[0] / root);
        }
        float total = 0.0f;
        for (int j = 0; j < nsplit; j++) {
            float ss = 0.0f;
            for (int t = j * ORC_ATT32_SPLIT; t < n_tok && t < (j + 1) * ORC_ATT32_SPLIT; t++) ss = ss + e[t];
            total = total + ss;
        }
        for (int d = 0; d < head_dim; d++) {
            float o = 0.0f;
            for (int j = 0; j < nsplit; j++) {
                float part = 0.0f;
                for (int t = j * ORC_ATT32_SPLIT; t < n_tok && t < (j + 1) * ORC_ATT32_SPLIT; t++) {
                    const float p = e[t] / total;
                    const float pv = p * vcache[((size_t)t * n_heads + h) * head_dim + d];
                    part = part + pv;
                }
                o = o + part;
            }
            out[(size_t)h * head_dim + d] = o;
        }
        free(e);
        free(lp);
    }
}

/* The reference's KV append for its own cache layout (attention.hpp:172-189,
 * :281-309): RoPE of k (rope_mx on the repeated heads; every repeat of a KV
 * head has the same values), then K and V of KV head h / rep stored for
 * every query head h at position pos, fp32 [n_heads][head_dim]; q rotated
 * into q_out. */
void orc_rope_kv_rep32(const float* q, const float* k, const float* v, const float* table_row,
                       int n_heads, int n_kv, int head_dim, float* q_out, float* k_row, float* v_row)
{
    int rep = n_heads / n_kv;
    float* kr = (float*)malloc(sizeof(float) * (size_t)n_kv * head_dim);
    orc_rope(q, table_row, n_heads, head_dim, q_out);
    orc_rope(k, table_row, n_kv, head_dim, kr);
    for (int h = 0; h < n_heads; h++) {
        memcpy(k_row + (size_t)h * head_dim, kr + (size_t)(h / rep) * head_dim, sizeof(float) * (size_t)head_dim);
        memcpy(v_row + (size_t)h * head_dim, v + (size_t)(h / rep) * head_dim, sizeof(float) * (size_t)head_dim);
    }
    free(kr);
}

/* matmul16x32 (aux.cl:454-490, called with 256 work-items per row at
 * model.hpp:207-227): row r of the dense fp16 matrix times x.  Work-item l
 * of the row sums w[l + 256k] * x[l + 256k] over k in order (a fp32 product,
 * then a fp32 add: no contraction), then the 256 partial sums go through the
 * work-group tree (stride 128 down to 1: p[l] += p[l + stride]). */
void orc_matmul_f16_dense(const uint16_t* W, const float* x, int rows, int cols, float* out)
{
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        float part[ORC_DENSE_WG];
        const uint16_t* w = W + (size_t)r * cols;
        for (int l = 0; l < ORC_DENSE_WG; l++) {
            float s = 0.0f;
            for (int i = l; i < cols; i += ORC_DENSE_WG) {
                const float pr = orc_f16_to_f32(w[i]) * x[i];
                s = s + pr;
            }
            part[l] = s;
        }
        for (int st = ORC_DENSE_WG / 2; st > 0; st >>= 1)
            for (int l = 0; l < st; l++) part[l] = part[l] + part[l + st];
        out[r] = part[0];
    }
}

int orc_argmax(const float* v, int n)
{
    int best = 0;
    for (int i = 1; i < n; i++)
        if (v[i] > v[best]) best = i;
    return best;
}

/* ------------------------------------------------------------------------- */
/* model                                                                      */
/* ------------------------------------------------------------------------- */

static void mat_apply(const orc_matrix* w, const float* x, float effort, float* y)
{
    int C = w->out_dim / 16;
    int R = w->in_dim * 16;
    orc_bucketmul(x, w->stats, w->probes, w->buckets, 0, w->in_dim, C, R, effort, y, NULL,
                  NULL, 1);
}

/* TransformerLayer::forward (transformer_layer.hpp:75-122) with
 * Attention::forward (attention.hpp:135-202) and FeedForward::run_forward
 * (feedforward.hpp:46-86); the KV cache is fp16 GQA [max_ctx][n_kv][hd]. */
void orc_layer_forward(const orc_model* m, int layer, int pos, float effort, float* h)
{
    const orc_model_config* c = &m->cfg;
    const orc_layer* L = &m->layers[layer];
    const int D = c->dim, F = c->ffn_dim, HD = c->head_dim;
    const int KVD = c->n_kv_heads * HD;
    float* hn = (float*)malloc(sizeof(float) * (size_t)D);
    float* q = (float*)malloc(sizeof(float) * (size_t)D);
    float* k = (float*)malloc(sizeof(float) * (size_t)KVD);
    float* v = (float*)malloc(sizeof(float) * (size_t)KVD);
    float* qr = (float*)malloc(sizeof(float) * (size_t)D);
    float* kr = (float*)malloc(sizeof(float) * (size_t)KVD);
    float* att = (float*)malloc(sizeof(float) * (size_t)D);
    float* o = (float*)malloc(sizeof(float) * (size_t)D);
    float* g = (float*)malloc(sizeof(float) * (size_t)F);
    float* u = (float*)malloc(sizeof(float) * (size_t)F);
    float* s = (float*)malloc(sizeof(float) * (size_t)F);

    orc_rmsnorm_gain(h, L->attn_gain, D, c->norm_eps, hn);
    mat_apply(&L->wq, hn, effort, q);
    mat_apply(&L->wk, hn, effort, k);
    mat_apply(&L->wv, hn, effort, v);
    const float* trow = m->rope + (size_t)pos * (HD / 2) * 2;
    orc_rope(q, trow, c->n_heads, HD, qr);
    orc_rope(k, trow, c->n_kv_heads, HD, kr);
    size_t lay = (size_t)layer * (size_t)c->max_ctx * (size_t)KVD;
    uint16_t* kc = m->kcache + lay;
    uint16_t* vc = m->vcache + lay;
    orc_f32_to_f16_n(kr, kc + (size_t)pos * KVD, (size_t)KVD);
    orc_f32_to_f16_n(v, vc + (size_t)pos * KVD, (size_t)KVD);
    orc_attention_f16kv(qr, kc, vc, pos + 1, c->n_heads, c->n_kv_heads, HD, att);
    mat_apply(&L->wo, att, effort, o);
    orc_add(h, o, D, h);
    orc_rmsnorm_gain(h, L->ffn_gain, D, c->norm_eps, hn);
    mat_apply(&L->w1, hn, effort, g);
    mat_apply(&L->w3, hn, effort, u);
    orc_silu_mul(g, u, F, s);
    mat_apply(&L->w2, s, effort, o);
    orc_add(h, o, D, h);

    free(hn); free(q); free(k); free(v); free(qr); free(kr);
    free(att); free(o); free(g); free(u); free(s);
}

/* MistralModel::forward, model.hpp:152-231; the LM head is the reference's
 * dense matmul16x32 when m->lm_dense is set, otherwise the bucket layout at
 * the same effort. */
void orc_model_forward(const orc_model* m, int token, int pos, float effort,
                       const float* hidden_in, float* logits)
{
    const orc_model_config* c = &m->cfg;
    float* h = (float*)malloc(sizeof(float) * (size_t)c->dim);
    float* hn = (float*)malloc(sizeof(float) * (size_t)c->dim);
    if (hidden_in) memcpy(h, hidden_in, sizeof(float) * (size_t)c->dim);
    else orc_embed(m->embed, c->dim, token, h);
    for (int l = 0; l < c->n_layers; l++) orc_layer_forward(m, l, pos, effort, h);
    orc_rmsnorm_gain(h, m->final_gain, c->dim, c->norm_eps, hn);
    if (m->lm_dense) orc_matmul_f16_dense(m->lm_dense, hn, c->vocab, c->dim, logits);
    else mat_apply(&m->lm_head, hn, effort, logits);
    free(h);
    free(hn);
}

/* threads the parallel loops above use (OpenMP's maximum; 1 without it) */
int orc_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
