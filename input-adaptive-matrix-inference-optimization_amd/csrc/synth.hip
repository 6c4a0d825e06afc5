// Synthetic weights and the bucket-layout producer on the GPU.
//
// Generator: element n of tensor `tid` = mean + sigma * N, with
// N = (sum of 12 uniform uint32 - 6*2^32) / 2^32 drawn from a counter-based
// splitmix64 stream keyed by (seed, tid).  Integer sums and power-of-two
// scaling are exact, the affine map uses explicitly rounded double ops and
// the result is rounded once (to fp16 or to float), so the bytes equal the
// CPU generator's on any machine.
//
// Bucketizer: bucketize_fp16_packed (preprocess_layer_fixed_gpu.py:110-242)
// with its exact numerics:
//   probes  fp16(float32 sum over j of |W[j,i]| in j order / out_dim) (:145, :154)
//   buckets rows i*16 + rank, |w| descending within each bucket of 16, ties in
//           original order (:163-188); code = (fp16 bits & 0xFFF0) | position (:192-200)
//   stats   fp16(numpy pairwise float32 sum of the row's |values| / nb),
//           replicated into 4 channels (:211-221)
#include <hip/hip_fp16.h>

#include "internal.h"
#include "layer_ops.h"

namespace iam {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ULL;

__host__ __device__ inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

static uint64_t stream_key(uint64_t seed, uint64_t tid)
{
    return mix64(mix64(seed + kGolden) ^ (tid * 0xD1B54A32D192ED03ULL));
}

__device__ inline double gen_normal(uint64_t key, uint64_t n)
{
    uint64_t s = 0;
#pragma unroll
    for (int j = 0; j < 6; j++) {
        const uint64_t u = mix64(key + (n * 6 + (uint64_t)j + 1) * kGolden);
        s += (u & 0xffffffffULL) + (u >> 32);
    }
    const int64_t c = (int64_t)s - (int64_t)(6ULL << 32);
    return (double)c * (1.0 / 4294967296.0);
}

__global__ void k_gen_f16(uint64_t key, size_t count, double mean, double sigma, uint16_t* __restrict__ out)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < count; i += stride) {
        const double v = __dadd_rn(mean, __dmul_rn(sigma, gen_normal(key, i)));
        const _Float16 h = static_cast<_Float16>(v);   // one rounding, double -> fp16
        out[i] = __builtin_bit_cast(uint16_t, h);
    }
}

__global__ void k_gen_f32(uint64_t key, size_t count, double mean, double sigma, float* __restrict__ out)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < count; i += stride) {
        const double v = __dadd_rn(mean, __dmul_rn(sigma, gen_normal(key, i)));
        out[i] = __double2float_rn(v);
    }
}

__device__ __forceinline__ float h2f(uint16_t b) { return __half2float(__ushort_as_half(b)); }

// probes: one thread per input column, float32 sum in j order
__global__ void k_probes(const uint16_t* __restrict__ W, int out_dim, int in_dim, uint16_t* __restrict__ probes)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= in_dim) return;
    float acc = 0.0f;
    int j = 0;
    for (; j + 8 <= out_dim; j += 8) {
        uint16_t v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = W[(size_t)(j + u) * in_dim + i];
#pragma unroll
        for (int u = 0; u < 8; u++) acc = __fadd_rn(acc, fabsf(h2f(v[u])));
    }
    for (; j < out_dim; j++) acc = __fadd_rn(acc, fabsf(h2f(W[(size_t)j * in_dim + i])));
    probes[i] = __half_as_ushort(__float2half_rn(__fdiv_rn(acc, (float)out_dim)));
}

// sort within each bucket of 16: rank_p = #{q : |w_q| > |w_p|} + #{q < p : |w_q| == |w_p|}
__global__ void k_bucket_sort(const uint16_t* __restrict__ W, int in_dim, int nb, uint16_t* __restrict__ buckets)
{
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)in_dim * nb) return;
    const int i = (int)(idx % in_dim);
    const int b = (int)(idx / in_dim);
    uint16_t v[16];
    float key[16];
#pragma unroll
    for (int p = 0; p < 16; p++) v[p] = W[(size_t)(b * 16 + p) * in_dim + i];
#pragma unroll
    for (int p = 0; p < 16; p++) key[p] = fabsf(h2f(v[p]));
#pragma unroll
    for (int p = 0; p < 16; p++) {
        int rank = 0;
#pragma unroll
        for (int q = 0; q < 16; q++) rank += (key[q] > key[p]) || (key[q] == key[p] && q < p);
        buckets[((size_t)i * 16 + rank) * nb + b] = (uint16_t)((v[p] & 0xFFF0u) | (unsigned)p);
    }
}

// |original value| of row r = (i, rank) in bucket b: the position bits of the
// packed code point back at W
struct RowValues {
    const uint16_t* W;
    const uint16_t* brow;
    int in_dim, i;
    __device__ float operator()(int b) const
    {
        const int p = brow[b] & 15;
        return fabsf(h2f(W[(size_t)(b * 16 + p) * in_dim + i]));
    }
};

template <typename F>
__device__ float pw_leaf(const F& f, int a, int n)
{
    if (n < 8) {
        float res = -0.0f;
        for (int i = 0; i < n; i++) res = __fadd_rn(res, f(a + i));
        return res;
    }
    float r[8];
#pragma unroll
    for (int j = 0; j < 8; j++) r[j] = f(a + j);
    int i = 8;
    for (; i < n - (n % 8); i += 8) {
#pragma unroll
        for (int j = 0; j < 8; j++) r[j] = __fadd_rn(r[j], f(a + i + j));
    }
    float res = __fadd_rn(__fadd_rn(__fadd_rn(r[0], r[1]), __fadd_rn(r[2], r[3])),
                          __fadd_rn(__fadd_rn(r[4], r[5]), __fadd_rn(r[6], r[7])));
    for (; i < n; i++) res = __fadd_rn(res, f(a + i));
    return res;
}

// numpy's pairwise summation (blocks of <= 128, split at n/2 rounded down to
// a multiple of 8), evaluated with an explicit stack
template <typename F>
__device__ float pairwise_sum(const F& f, int n)
{
    struct Frame {
        int a, n, state;
        float left;
    };
    Frame st[24];
    int sp = 0;
    st[0] = {0, n, 0, 0.0f};
    float result = 0.0f;
    while (sp >= 0) {
        Frame& fr = st[sp];
        if (fr.n <= 128) {
            result = pw_leaf(f, fr.a, fr.n);
            sp--;
            continue;
        }
        int n2 = fr.n / 2;
        n2 -= n2 % 8;
        if (fr.state == 0) {
            fr.state = 1;
            st[sp + 1] = {fr.a, n2, 0, 0.0f};
            sp++;
        } else if (fr.state == 1) {
            fr.left = result;
            fr.state = 2;
            st[sp + 1] = {fr.a + n2, fr.n - n2, 0, 0.0f};
            sp++;
        } else {
            result = __fadd_rn(fr.left, result);
            sp--;
        }
    }
    return result;
}

__global__ void k_bucket_stats(const uint16_t* __restrict__ W, const uint16_t* __restrict__ buckets, int in_dim,
                               int nb, uint16_t* __restrict__ stats)
{
    const size_t r = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= (size_t)in_dim * 16) return;
    RowValues f{W, buckets + r * nb, in_dim, (int)(r / 16)};
    const float s = __fadd_rn(0.0f, pairwise_sum(f, nb));
    const uint16_t m = __half_as_ushort(__float2half_rn(__fdiv_rn(s, (float)nb)));
    const uint32_t m2 = (uint32_t)m | ((uint32_t)m << 16);
    reinterpret_cast<uint2*>(stats)[r] = make_uint2(m2, m2);
}

static unsigned grid_for(size_t n, unsigned block, unsigned cap = 65535u * 4)
{
    size_t g = (n + block - 1) / block;
    return (unsigned)(g < cap ? (g ? g : 1) : cap);
}

int gen_f16(Ctx* c, uint64_t seed, uint64_t tid, size_t count, double mean, double sigma, uint16_t* out)
{
    return launch(c, "gen_f16", k_gen_f16, dim3(grid_for(count, 256)), dim3(256), 0, stream_key(seed, tid), count,
                  mean, sigma, out);
}

int gen_f32(Ctx* c, uint64_t seed, uint64_t tid, size_t count, double mean, double sigma, float* out)
{
    return launch(c, "gen_f32", k_gen_f32, dim3(grid_for(count, 256)), dim3(256), 0, stream_key(seed, tid), count,
                  mean, sigma, out);
}

int bucketize(Ctx* c, const uint16_t* w, int out_dim, int in_dim, uint16_t* buckets, uint16_t* stats,
              uint16_t* probes)
{
    const int nb = out_dim / 16;
    IAM_TRY(launch(c, "bucketize_probes", k_probes, dim3((in_dim + 255) / 256), dim3(256), 0, w, out_dim, in_dim,
                   probes));
    const size_t ncol = (size_t)in_dim * nb;
    IAM_TRY(launch(c, "bucketize_sort", k_bucket_sort, dim3((unsigned)((ncol + 255) / 256)), dim3(256), 0, w,
                   in_dim, nb, buckets));
    const size_t rows = (size_t)in_dim * 16;
    return launch(c, "bucketize_stats", k_bucket_stats, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, w,
                  (const uint16_t*)buckets, in_dim, nb, stats);
}

}  // namespace iam

using namespace iam;

extern "C" {

int iam_gen_f16(iam_ctx* c, uint64_t seed, uint64_t tid, size_t count, double mean, double sigma, uint16_t* out)
{
    if (!c || !out) return fail(IAM_E_INVALID, "gen_f16: null argument");
    if (count == 0) return IAM_OK;
    IAM_TRY(check_dev_range(c, out, count * 2, "gen_f16 out"));
    return gen_f16(c, seed, tid, count, mean, sigma, out);
}

int iam_gen_f32(iam_ctx* c, uint64_t seed, uint64_t tid, size_t count, double mean, double sigma, float* out)
{
    if (!c || !out) return fail(IAM_E_INVALID, "gen_f32: null argument");
    if (count == 0) return IAM_OK;
    IAM_TRY(check_dev_range(c, out, count * 4, "gen_f32 out"));
    return gen_f32(c, seed, tid, count, mean, sigma, out);
}

int iam_bucketize(iam_ctx* c, const uint16_t* w, int out_dim, int in_dim, uint16_t* buckets, uint16_t* stats,
                  uint16_t* probes)
{
    if (!c || !w || !buckets || !stats || !probes) return fail(IAM_E_INVALID, "bucketize: null argument");
    IAM_REQUIRE(out_dim > 0 && in_dim > 0 && out_dim % 16 == 0,
                "bucketize: out_dim must be a positive multiple of 16");
    const size_t n = (size_t)out_dim * in_dim;
    IAM_TRY(check_dev_range(c, w, n * 2, "bucketize W"));
    IAM_TRY(check_dev_range(c, buckets, n * 2, "bucketize buckets"));
    IAM_TRY(check_dev_range(c, stats, (size_t)in_dim * 16 * 4 * 2, "bucketize stats"));
    IAM_TRY(check_dev_range(c, probes, (size_t)in_dim * 2, "bucketize probes"));
    IAM_REQUIRE((((uintptr_t)stats) & 7) == 0, "bucketize: stats must be 8-byte aligned");
    return bucketize(c, w, out_dim, in_dim, buckets, stats, probes);
}

}  // extern "C"
