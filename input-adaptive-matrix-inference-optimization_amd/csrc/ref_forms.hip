// The reference's own fp32 forms, for callers that need its numbers rather
// than the decode step's faster ones:
//   - its KV cache layout (K and V repeated to every query head, fp32
//     [max_ctx][n_heads][head_dim] per layer, model.hpp:97-98) with the
//     RoPE + append of attention.hpp:172-189 / :281-309 and its fp32
//     attention (dotSetScore2, sum_of_exps32_mx, softmax_add32_mx,
//     sumScores32: aux.cl:204-225, :370-384, :497-540);
//   - its dense fp16 LM head, matmul16x32 (aux.cl:454-490, model.hpp:207-227).
// Every fp32 operation is a single IEEE-rounded one (no contraction), in the
// reference's order where that order is fixed; where the reference's order
// depends on scheduling (the float atomics of sum_of_exps32_mx) a fixed one
// is used.  The results then equal the oracle's restatement of the same
// order (exp excepted: the device's expf may differ from the C library's by
// an ulp).
#include <hip/hip_fp16.h>

#include <algorithm>
#include <cmath>

#include "internal.h"
#include "layer_ops.h"

namespace iam {

namespace {

__device__ __forceinline__ float f16(uint32_t bits) { return __half2float(__ushort_as_half((unsigned short)(bits & 0xffffu))); }

constexpr int kSplit = 64;        // positions per split of the fp32 attention
constexpr int kHD = 128;          // head dimension
constexpr int kDenseWG = 256;     // work-items per row of matmul16x32 (model.hpp:223-224)

}  // namespace

// ---------------------------------------------------------------- append ---
// RoPE of q (n_heads heads) and of k (n_kv heads), then the K row after RoPE
// and the V row of KV head h / rep stored for every query head h at the
// position (repeat4x32 + rope_mx + the cache copies).
__global__ void k_rope_kv_rep32(const float* __restrict__ q, const float* __restrict__ k,
                                const float* __restrict__ v, const float* __restrict__ table,
                                const int* __restrict__ pos_p, int n_heads, int n_kv, int max_ctx,
                                float* __restrict__ q_out, float* __restrict__ kc, float* __restrict__ vc)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int pos = *pos_p;
    if (pos < 0 || pos >= max_ctx) return;
    const int nq = n_heads * kHD;
    const int rep = n_heads / n_kv;
    const float* row = table + (size_t)pos * kHD;
    if (i < nq) {
        const int h = i / kHD, d = i - h * kHD;
        q_out[i] = rope_one(q + h * kHD, row, d, kHD / 2);
    } else if (i < 2 * nq) {
        const int j = i - nq;
        const int h = j / kHD, d = j - h * kHD;
        kc[(size_t)pos * nq + j] = rope_one(k + (h / rep) * kHD, row, d, kHD / 2);
    } else if (i < 3 * nq) {
        const int j = i - 2 * nq;
        const int h = j / kHD, d = j - h * kHD;
        vc[(size_t)pos * nq + j] = v[(h / rep) * kHD + d];
    }
}

// ------------------------------------------------------------- attention ---
// Pass 1, workgroup (head h, split j) of 4 waves: the score of each position
// t of the split (wave w takes positions t0 + w, t0 + w + 4, ...) as
// dotSetScore2 forms it -- lane l multiplies dimensions l and l + 64, adds
// the two (the tree's stride 64), and the strides 32 .. 1 follow as
// shuffles, so the sum is the reference's work-group tree -- divided by
// sqrt(128); e_t = exp(s_t) (no maximum subtracted) goes to e[h][t].  The
// split's sum of e in position order goes to ssum[h][j].
__global__ __launch_bounds__(256) void k_att32_score(const float* __restrict__ q, const float* __restrict__ kc,
                                                     const int* __restrict__ pos_p, int n_heads, int max_ctx,
                                                     float* __restrict__ e, float* __restrict__ ssum)
{
#pragma clang fp contract(off)
    __shared__ float se[kSplit];
    const int h = blockIdx.x, j = blockIdx.y;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int n_tok = min(*pos_p + 1, max_ctx);
    const int t0 = j * kSplit;
    const int nt = min(kSplit, n_tok - t0);
    if (nt <= 0) return;
    const float root = __fsqrt_rn((float)kHD);
    const float q0 = q[h * kHD + lane], q1 = q[h * kHD + 64 + lane];
    for (int i = w; i < nt; i += 4) {
        const float* kr = kc + ((size_t)(t0 + i) * n_heads + h) * kHD;
        float a = __fadd_rn(__fmul_rn(q0, kr[lane]), __fmul_rn(q1, kr[64 + lane]));
#pragma unroll
        for (int st = 32; st > 0; st >>= 1) a = __fadd_rn(a, __shfl_down(a, st, 64));
        if (lane == 0) {
            const float ev = expf(__fdiv_rn(a, root));
            se[i] = ev;
            e[(size_t)h * max_ctx + t0 + i] = ev;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float s = 0.0f;
        for (int i = 0; i < nt; i++) s = __fadd_rn(s, se[i]);
        ssum[(size_t)h * gridDim.y + j] = s;
    }
}

// Pass 2, workgroup (head h, split j), thread d: the total of the splits'
// sums in split order, p_t = e_t / total (softmax_add32_mx), and the split's
// sum of p_t * v_t[d] in position order (sumScores32's products) into
// part[h][j][d].
__global__ __launch_bounds__(kHD) void k_att32_pv(const float* __restrict__ vc, const int* __restrict__ pos_p,
                                                  int n_heads, int max_ctx, const float* __restrict__ e,
                                                  const float* __restrict__ ssum, float* __restrict__ part)
{
#pragma clang fp contract(off)
    __shared__ float sp[kSplit];
    const int h = blockIdx.x, j = blockIdx.y, d = threadIdx.x;
    const int n_tok = min(*pos_p + 1, max_ctx);
    const int t0 = j * kSplit;
    const int nt = min(kSplit, n_tok - t0);
    if (nt <= 0) return;
    const int ns = (n_tok + kSplit - 1) / kSplit;
    float total = 0.0f;
    for (int s = 0; s < ns; s++) total = __fadd_rn(total, ssum[(size_t)h * gridDim.y + s]);
    if (d < nt) sp[d] = __fdiv_rn(e[(size_t)h * max_ctx + t0 + d], total);
    __syncthreads();
    float acc = 0.0f;
    for (int i = 0; i < nt; i++)
        acc = __fadd_rn(acc, __fmul_rn(sp[i], vc[((size_t)(t0 + i) * n_heads + h) * kHD + d]));
    part[((size_t)h * gridDim.y + j) * kHD + d] = acc;
}

// Pass 3, workgroup h, thread d: out[h][d] = the splits' sums in split order.
__global__ __launch_bounds__(kHD) void k_att32_sum(const int* __restrict__ pos_p, int max_ctx, int nsplit,
                                                   const float* __restrict__ part, float* __restrict__ out)
{
#pragma clang fp contract(off)
    const int h = blockIdx.x, d = threadIdx.x;
    const int n_tok = min(*pos_p + 1, max_ctx);
    const int ns = n_tok > 0 ? (n_tok + kSplit - 1) / kSplit : 0;
    float o = 0.0f;
    for (int s = 0; s < ns; s++) o = __fadd_rn(o, part[((size_t)h * nsplit + s) * kHD + d]);
    out[(size_t)h * kHD + d] = o;
}

// ----------------------------------------------------------------- dense ---
// matmul16x32 with 256 work-items per row: work-item l of a row sums the
// products of columns l, l + 256, ... in order, then the 256 partial sums
// go through the tree p[l] += p[l + stride], stride 128 .. 1.  Here one
// wave holds a row's 256 work-items, lane i the four l = 4i .. 4i + 3 (one
// 8-byte load per 256 columns); the tree's strides 128 .. 4 are shuffles
// between lanes 32 .. 1 apart, strides 2 and 1 stay in lane 0.  x is staged
// in LDS; each wave walks rows wave, wave + waves, ... two at a time.
constexpr int kDenseThreads = 256;
constexpr int kDenseMaxCols = 16384;

template <bool VEC>
__global__ __launch_bounds__(kDenseThreads) void k_matmul16x32(const uint16_t* __restrict__ W,
                                                               const float* __restrict__ x, int rows, int cols,
                                                               float* __restrict__ out)
{
#pragma clang fp contract(off)
    extern __shared__ __align__(16) float sx[];   // x, cols floats
    for (int i = threadIdx.x; i < cols; i += kDenseThreads) sx[i] = x[i];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int waves = gridDim.x * (kDenseThreads / 64);
    const int wv = blockIdx.x * (kDenseThreads / 64) + (threadIdx.x >> 6);
    const int nk = (cols + kDenseWG - 1) / kDenseWG;
    auto row_sums = [&](int r, float (&s)[4]) {
        const uint16_t* w = W + (size_t)r * cols;
#pragma unroll
        for (int c = 0; c < 4; c++) s[c] = 0.0f;
        for (int k = 0; k < nk; k++) {
            const int b = k * kDenseWG + 4 * lane;
            uint32_t v[4];
            if (VEC && b + 3 < cols) {
                typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
                const u32x2 p = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(w + b));
                v[0] = p.x;
                v[1] = p.x >> 16;
                v[2] = p.y;
                v[3] = p.y >> 16;
            } else {
#pragma unroll
                for (int c = 0; c < 4; c++) v[c] = b + c < cols ? (uint32_t)w[b + c] : 0u;
            }
#pragma unroll
            for (int c = 0; c < 4; c++)
                if (b + c < cols) s[c] = __fadd_rn(s[c], __fmul_rn(f16(v[c]), sx[b + c]));
        }
    };
    auto tree = [&](float (&s)[4]) -> float {
#pragma unroll
        for (int st = 32; st > 0; st >>= 1) {
#pragma unroll
            for (int c = 0; c < 4; c++) s[c] = __fadd_rn(s[c], __shfl_down(s[c], st, 64));
        }
        const float a0 = __fadd_rn(s[0], s[2]), a1 = __fadd_rn(s[1], s[3]);
        return __fadd_rn(a0, a1);
    };
    for (int r = wv; r < rows; r += 2 * waves) {
        float s0[4], s1[4];
        const int r1 = r + waves;
        row_sums(r, s0);
        if (r1 < rows) row_sums(r1, s1);
        const float y0 = tree(s0);
        if (lane == 0) out[r] = y0;
        if (r1 < rows) {
            const float y1 = tree(s1);
            if (lane == 0) out[r1] = y1;
        }
    }
}

}  // namespace iam

using namespace iam;

int iam::ensure_attn32_scratch(Ctx* c, size_t floats)
{
    if (floats <= c->attn32_cap && c->attn32) return IAM_OK;
    if (c->capturing) return fail(IAM_E_STATE, "fp32 attention scratch growth during graph capture");
    if (c->attn32) IAM_TRY(ctx_free(c, c->attn32));
    c->attn32 = nullptr;
    c->attn32_cap = 0;
    IAM_TRY(ctx_alloc(c, floats * sizeof(float), (void**)&c->attn32));
    c->attn32_cap = floats;
    c->scratch_gen++;
    return IAM_OK;
}

int iam::matmul_f16_dense(Ctx* c, const uint16_t* W, const float* x, int rows, int cols, float* out)
{
    const int waves_needed = (rows + 1) / 2;
    const int blocks = std::max(1, std::min(2048, (waves_needed + 3) / 4));
    const bool vec = (cols % 4) == 0 && ((uintptr_t)W & 7) == 0;
    const size_t lds = (size_t)cols * sizeof(float);
    if (vec)
        return launch(c, "matmul16x32", k_matmul16x32<true>, dim3(blocks), dim3(kDenseThreads), lds, W, x, rows,
                      cols, out);
    return launch(c, "matmul16x32", k_matmul16x32<false>, dim3(blocks), dim3(kDenseThreads), lds, W, x, rows, cols,
                  out);
}

extern "C" {

int iam_rope_kv_append_f32(iam_ctx* c, const float* q, const float* k, const float* v, const float* table,
                           const int* pos, int n_heads, int n_kv, int head_dim, int max_ctx, float* q_out,
                           float* kc, float* vc)
{
    if (!c || !q || !k || !v || !table || !pos || !q_out || !kc || !vc)
        return fail(IAM_E_INVALID, "rope_kv_append_f32: null argument");
    IAM_REQUIRE(head_dim == kHD, "rope_kv_append_f32: head_dim must be 128");
    IAM_REQUIRE(n_kv > 0 && n_heads >= n_kv && n_heads % n_kv == 0 && max_ctx > 0,
                "rope_kv_append_f32: n_heads must be a positive multiple of n_kv");
    const size_t nq = (size_t)n_heads * kHD, nk = (size_t)n_kv * kHD;
    IAM_TRY(check_dev_range(c, q, nq * 4, "rope_kv_f32 q"));
    IAM_TRY(check_dev_range(c, k, nk * 4, "rope_kv_f32 k"));
    IAM_TRY(check_dev_range(c, v, nk * 4, "rope_kv_f32 v"));
    IAM_TRY(check_dev_range(c, q_out, nq * 4, "rope_kv_f32 q_out"));
    IAM_TRY(check_dev_range(c, table, (size_t)max_ctx * kHD * 4, "rope_kv_f32 table"));
    IAM_TRY(check_dev_range(c, kc, (size_t)max_ctx * nq * 4, "rope_kv_f32 kcache"));
    IAM_TRY(check_dev_range(c, vc, (size_t)max_ctx * nq * 4, "rope_kv_f32 vcache"));
    IAM_TRY(check_dev_range(c, pos, 4, "rope_kv_f32 pos"));
    const int n = 3 * (int)nq;
    return launch(c, "rope_kv_append_f32", k_rope_kv_rep32, dim3((n + 255) / 256), dim3(256), 0, q, k, v, table,
                  pos, n_heads, n_kv, max_ctx, q_out, kc, vc);
}

int iam_attention_decode_f32(iam_ctx* c, const float* q, const float* kc, const float* vc, const int* pos,
                             int n_heads, int head_dim, int max_ctx, float* out)
{
    if (!c || !q || !kc || !vc || !pos || !out) return fail(IAM_E_INVALID, "attention_f32: null argument");
    IAM_REQUIRE(head_dim == kHD, "attention_f32: head_dim must be 128");
    IAM_REQUIRE(n_heads >= 1 && n_heads <= 1024, "attention_f32: n_heads must be in [1, 1024]");
    IAM_REQUIRE(max_ctx >= 1 && max_ctx <= (1 << 20), "attention_f32: max_ctx must be in [1, 2^20]");
    const size_t nq = (size_t)n_heads * kHD;
    IAM_TRY(check_dev_range(c, q, nq * 4, "attention_f32 q"));
    IAM_TRY(check_dev_range(c, kc, (size_t)max_ctx * nq * 4, "attention_f32 kcache"));
    IAM_TRY(check_dev_range(c, vc, (size_t)max_ctx * nq * 4, "attention_f32 vcache"));
    IAM_TRY(check_dev_range(c, out, nq * 4, "attention_f32 out"));
    IAM_TRY(check_dev_range(c, pos, 4, "attention_f32 pos"));
    const int nsplit = (max_ctx + kSplit - 1) / kSplit;
    // scratch: e [n_heads][max_ctx], split sums [n_heads][nsplit], split partials [n_heads][nsplit][128]
    const size_t ne = (size_t)n_heads * max_ctx, ns = (size_t)n_heads * nsplit, np = ns * kHD;
    IAM_TRY(ensure_attn32_scratch(c, ne + ns + np));
    float* e = c->attn32;
    float* ssum = e + ne;
    float* part = ssum + ns;
    IAM_TRY(launch(c, "attention_f32.score", k_att32_score, dim3(n_heads, nsplit), dim3(256), 0, q, kc, pos, n_heads,
                   max_ctx, e, ssum));
    IAM_TRY(launch(c, "attention_f32.pv", k_att32_pv, dim3(n_heads, nsplit), dim3(kHD), 0, vc, pos, n_heads, max_ctx,
                   (const float*)e, (const float*)ssum, part));
    return launch(c, "attention_f32.sum", k_att32_sum, dim3(n_heads), dim3(kHD), 0, pos, max_ctx, nsplit,
                  (const float*)part, out);
}

int iam_matmul_f16_dense(iam_ctx* c, const uint16_t* W, const float* x, int rows, int cols, float* out)
{
    if (!c || !W || !x || !out) return fail(IAM_E_INVALID, "matmul_f16_dense: null argument");
    IAM_REQUIRE(rows >= 1 && cols >= 1 && cols <= kDenseMaxCols, "matmul_f16_dense: rows >= 1, 1 <= cols <= 16384");
    IAM_TRY(check_dev_range(c, W, (size_t)rows * cols * 2, "matmul_f16_dense W"));
    IAM_TRY(check_dev_range(c, x, (size_t)cols * 4, "matmul_f16_dense x"));
    IAM_TRY(check_dev_range(c, out, (size_t)rows * 4, "matmul_f16_dense out"));
    return matmul_f16_dense(c, W, x, rows, cols, out);
}

}  // extern "C"
