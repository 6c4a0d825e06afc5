// Mistral-shaped decoder over the bucket-layout weights.
//
// MistralModel::forward (model.hpp:152-231) = embedding gather, 32 x
// TransformerLayer::forward (transformer_layer.hpp:75-122: norm -> attention
// -> +res -> norm -> FFN -> +res), final norm, LM head, greedy argmax
// (test_generation.cpp:235/276).  Differences that are the point of the
// build: q/k/v and gate/up run as one walk launch and one reduce launch per
// group; the walk computes the RMSNorm of its input and the cutoff itself;
// the reduce applies the residual add, RoPE with the fp16 KV append, or the
// SiLU gate to its sums; attention is split over the context (partials, then
// their merge); the position and token live in device memory, so a whole
// step is captured once as a HIP graph and replayed per token with no host
// round trip.
#include <hip/hip_fp16.h>

#include <cstring>
#include <string>
#include <vector>

#include "internal.h"
#include "layer_ops.h"

namespace iam {

struct Mat {
    uint16_t* buckets = nullptr;
    uint16_t* stats = nullptr;    // reference layout [R][4]
    uint16_t* stats3 = nullptr;   // compact channel 3 [R]
    uint16_t* probes = nullptr;   // [in_dim]
    int in_dim = 0, out_dim = 0;
    iam_bucket_matrix desc() const
    {
        return iam_bucket_matrix{buckets, stats3, probes, in_dim * 16, out_dim / 16, 1, 0};
    }
};

struct Layer {
    Mat wq, wk, wv, wo, w1, w3, w2;
    uint16_t* attn_gain = nullptr;
    uint16_t* ffn_gain = nullptr;
};

}  // namespace iam

struct iam_model {
    iam_ctx* c = nullptr;
    iam_model_config cfg{};
    std::vector<iam::Layer> layers;
    uint16_t* embed = nullptr;
    uint16_t* final_gain = nullptr;
    iam::Mat lm;
    uint16_t* kcache = nullptr;
    uint16_t* vcache = nullptr;
    float* rope = nullptr;
    float* embed_scale = nullptr;   // optional per-channel scale of the gathered embedding
    bool use_scale = false;
    // activations
    float *h = nullptr, *hn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *qr = nullptr;
    float *att = nullptr, *o = nullptr, *g = nullptr, *u = nullptr, *s = nullptr, *d = nullptr;
    float* logits = nullptr;
    int* token = nullptr;
    int* pos = nullptr;
    int* hist = nullptr;             // token history [max_ctx + 1]
    // captured step
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    float graph_effort = -1.0f;
    bool graph_override = false;
    uint64_t graph_gen = 0;          // Ctx::scratch_gen at capture
    std::vector<void*> owned;
};

namespace iam {

static int alloc_owned(iam_model* m, size_t bytes, void** p)
{
    IAM_TRY(ctx_alloc(m->c, bytes, p));
    m->owned.push_back(*p);
    return IAM_OK;
}

template <typename T>
static int alloc_t(iam_model* m, size_t n, T** p)
{
    return alloc_owned(m, n * sizeof(T), (void**)p);
}

static int alloc_mat(iam_model* m, Mat& w, int out_dim, int in_dim)
{
    w.in_dim = in_dim;
    w.out_dim = out_dim;
    const size_t R = (size_t)in_dim * 16;
    IAM_TRY(alloc_t(m, (size_t)out_dim * in_dim, &w.buckets));
    IAM_TRY(alloc_t(m, R * 4, &w.stats));
    IAM_TRY(alloc_t(m, R, &w.stats3));
    // probes padded to the 4096 values the cutoff always reads
    IAM_TRY(alloc_t(m, (size_t)std::max(in_dim, kProbes), &w.probes));
    return IAM_OK;
}

__global__ void k_set_int(int* p, int v) { *p = v; }

__global__ void k_scale_vec(float* __restrict__ h, const float* __restrict__ s, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) h[i] = __fmul_rn(h[i], s[i]);
}

__global__ void k_copy_f32(const float* __restrict__ a, float* __restrict__ b, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) b[i] = a[i];
}

// argmax + token history + position advance for the device-driven step
__global__ __launch_bounds__(1024) void k_pick(const float* __restrict__ v, int n, int* __restrict__ tok,
                                               int* __restrict__ pos, int* __restrict__ hist, int hist_len)
{
    __shared__ float sv[16];
    __shared__ int si[16];
    const int tid = threadIdx.x;
    float bv = -INFINITY;
    int bi = n;
    auto take = [&](float x, int i) {
        if (x > bv || (x == bv && i < bi)) {
            bv = x;
            bi = i;
        }
    };
    // 16-byte loads, 8 per thread in flight (the order of the candidates a
    // thread sees does not matter: ties go to the smaller index)
    const int n4 = (reinterpret_cast<uintptr_t>(v) & 15) == 0 ? n >> 2 : 0;
    const float4* v4 = reinterpret_cast<const float4*>(v);
    constexpr int U = 8;
    for (int b0 = 0; b0 < n4; b0 += U * 1024) {
        float4 r[U];
#pragma unroll
        for (int u = 0; u < U; u++) r[u] = v4[min(b0 + u * 1024 + tid, n4 - 1)];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int j = b0 + u * 1024 + tid;
            if (j < n4) {
                take(r[u].x, 4 * j);
                take(r[u].y, 4 * j + 1);
                take(r[u].z, 4 * j + 2);
                take(r[u].w, 4 * j + 3);
            }
        }
    }
    for (int i = 4 * n4 + tid; i < n; i += 1024) take(v[i], i);
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
        const int t = bi < n ? bi : 0;
        tok[0] = t;
        const int p = pos[0];
        if (p + 1 >= 0 && p + 1 < hist_len) hist[p + 1] = t;
        pos[0] = p + 1;
    }
}

// One matrix group through bucketmul_fused: x (in memory, or the norm of h
// written to x), cutoff, walk, reduce with the epilogues ep (null: store).
static int mat_group(iam_model* m, int n, const Mat* const* mats, float* x, int in_size, float* const* ys,
                     float effort, int in_mode, const float* h, const uint16_t* gain, const ReduceEp* ep)
{
    MatOp ops[kMaxMulti];
    for (int i = 0; i < n; i++) {
        ops[i].mat = mats[i]->desc();
        ops[i].x = x;
        ops[i].in_size = in_size;
        ops[i].y = ys[i];
    }
    return bucketmul_fused(m->c, n, ops, 0, effort, in_mode, h, gain, m->cfg.norm_eps, ep);
}

// One decode step reading token/pos from device memory.  logits_out may be
// the model's own buffer or a caller buffer of vocab floats.  Per layer:
//   q/k/v walk (attention norm of h fused in) -> reduce + RoPE + fp16 KV append
//   -> attention -> o walk -> reduce + residual (h += o)
//   -> w1/w3 walk (FFN norm of h fused in) -> reduce + SiLU gate
//   -> w2 walk -> reduce + residual (h += d)
// (transformer_layer.hpp:75-122, attention.hpp:135-202, feedforward.hpp:46-86).
static int step(iam_model* m, float effort, const float* hidden_override, float* logits_out, bool pick)
{
    Ctx* c = m->c;
    const iam_model_config& C = m->cfg;
    const int D = C.dim, F = C.ffn_dim;
    if (hidden_override) {
        IAM_TRY(launch(c, "copy_hidden", k_copy_f32, dim3((D + 255) / 256), dim3(256), 0, hidden_override, m->h, D));
    } else {
        IAM_TRY(embed(c, m->embed, D, C.vocab, m->token, m->h));
        if (m->use_scale)
            IAM_TRY(launch(c, "embed_scale", k_scale_vec, dim3((D + 255) / 256), dim3(256), 0, m->h,
                           (const float*)m->embed_scale, D));
    }
    const size_t kv_layer = (size_t)C.max_ctx * C.n_kv_heads * C.head_dim;
    for (int L = 0; L < C.n_layers; L++) {
        Layer& ly = m->layers[L];
        uint16_t* kc = m->kcache + (size_t)L * kv_layer;
        uint16_t* vc = m->vcache + (size_t)L * kv_layer;
        {
            const Mat* mats[3] = {&ly.wq, &ly.wk, &ly.wv};
            float* ys[3] = {m->q, m->k, m->v};
            ReduceEp ep[3];
            ep[0].ep = kEpRopeQ;
            ep[0].out = m->qr;
            ep[1].ep = kEpRopeK;
            ep[1].cache = kc;
            ep[2].ep = kEpV;
            ep[2].cache = vc;
            for (int i = 0; i < 3; i++) {
                ep[i].table = m->rope;
                ep[i].pos = m->pos;
                ep[i].max_ctx = C.max_ctx;
            }
            IAM_TRY(mat_group(m, 3, mats, m->hn, D, ys, effort, kInNorm, m->h, ly.attn_gain, ep));
        }
        IAM_TRY(attention(c, m->qr, kc, vc, m->pos, C.n_heads, C.n_kv_heads, C.max_ctx, c->attn_ws, m->att));
        {
            const Mat* mats[1] = {&ly.wo};
            float* ys[1] = {m->o};
            ReduceEp ep[1];
            ep[0].ep = kEpResid;
            ep[0].out = m->h;
            IAM_TRY(mat_group(m, 1, mats, m->att, D, ys, effort, kInX, nullptr, nullptr, ep));
        }
        {
            const Mat* mats[2] = {&ly.w1, &ly.w3};
            float* ys[2] = {m->g, m->u};
            ReduceEp ep[2];
            ep[0].ep = kEpSilu;
            ep[0].out = m->s;
            IAM_TRY(mat_group(m, 2, mats, m->hn, D, ys, effort, kInNorm, m->h, ly.ffn_gain, ep));
        }
        {
            const Mat* mats[1] = {&ly.w2};
            float* ys[1] = {m->d};
            ReduceEp ep[1];
            ep[0].ep = kEpResid;
            ep[0].out = m->h;
            IAM_TRY(mat_group(m, 1, mats, m->s, F, ys, effort, kInX, nullptr, nullptr, ep));
        }
    }
    {
        const Mat* mats[1] = {&m->lm};
        float* ys[1] = {logits_out};
        IAM_TRY(mat_group(m, 1, mats, m->hn, D, ys, effort, kInNorm, m->h, m->final_gain, nullptr));
    }
    if (pick)
        IAM_TRY(launch(c, "pick", k_pick, dim3(1), dim3(1024), 0, (const float*)logits_out, C.vocab, m->token,
                       m->pos, m->hist, C.max_ctx + 1));
    return IAM_OK;
}

// size the dispatch slots, walk partials and attention workspace for every
// matrix group of a step at this effort, so a step never allocates (which
// graph capture requires)
static int reserve(iam_model* m, float effort)
{
    Ctx* c = m->c;
    const iam_model_config& C = m->cfg;
    for (int s = 0; s < kMaxMulti; s++) IAM_TRY(ensure_slot(c, s));
    const Layer& ly = m->layers[0];
    const Mat* groups[5][3] = {{&ly.wq, &ly.wk, &ly.wv}, {&ly.wo}, {&ly.w1, &ly.w3}, {&ly.w2}, {&m->lm}};
    const int sizes[5] = {3, 1, 2, 1, 1};
    const int ins[5] = {C.dim, C.dim, C.dim, C.ffn_dim, C.dim};
    for (int gi = 0; gi < 5; gi++) {
        MatOp ops[kMaxMulti];
        for (int i = 0; i < sizes[gi]; i++) {
            ops[i].mat = groups[gi][i]->desc();
            ops[i].in_size = ins[gi];
        }
        IAM_TRY(reserve_walk(c, sizes[gi], ops, effort));
    }
    return ensure_attn_ws(c, attention_ws_floats(C.n_heads, C.max_ctx));
}

static int drop_graph(iam_model* m)
{
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    m->exec = nullptr;
    m->graph = nullptr;
    m->graph_effort = -1.0f;
    return IAM_OK;
}

static int capture_step(iam_model* m, float effort, bool override_hidden)
{
    Ctx* c = m->c;
    IAM_TRY(drop_graph(m));
    IAM_TRY(reserve(m, effort));
    IAM_CHECK_HIP(hipStreamSynchronize(c->stream));
    IAM_CHECK_HIP(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    c->capturing = true;
    int rc = step(m, effort, override_hidden ? m->s : nullptr, m->logits, true);
    c->capturing = false;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(c->stream, &g);
    if (rc != IAM_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) return fail(IAM_E_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(e));
    m->graph = g;
    IAM_CHECK_HIP(hipGraphInstantiate(&m->exec, g, nullptr, nullptr, 0));
    m->graph_effort = effort;
    m->graph_override = override_hidden;
    m->graph_gen = c->scratch_gen;
    return IAM_OK;
}

struct TensorRef {
    void* p;
    size_t bytes;
};

static bool lookup(iam_model* m, const std::string& name, TensorRef* out, const Mat** mat)
{
    const iam_model_config& C = m->cfg;
    const size_t D = C.dim, V = C.vocab;
    const size_t kv = (size_t)C.n_layers * C.max_ctx * C.n_kv_heads * C.head_dim * 2;
    auto matparts = [&](const Mat& w, const std::string& part) -> bool {
        const size_t R = (size_t)w.in_dim * 16;
        if (mat) *mat = &w;
        if (part == "buckets") *out = {w.buckets, (size_t)w.out_dim * w.in_dim * 2};
        else if (part == "stats") *out = {w.stats, R * 8};
        else if (part == "stats3") *out = {w.stats3, R * 2};
        else if (part == "probes") *out = {w.probes, (size_t)std::max(w.in_dim, kProbes) * 2};
        else if (part.empty()) *out = {w.buckets, (size_t)w.out_dim * w.in_dim * 2};
        else return false;
        return true;
    };
    auto split = [](const std::string& s, std::string& a, std::string& b) {
        size_t k = s.find('.');
        if (k == std::string::npos) {
            a = s;
            b.clear();
        } else {
            a = s.substr(0, k);
            b = s.substr(k + 1);
        }
    };
    std::string head, rest;
    split(name, head, rest);
    if (head == "embed") *out = {m->embed, V * D * 2};
    else if (head == "final_gain") *out = {m->final_gain, D * 2};
    else if (head == "lm_head") return matparts(m->lm, rest);
    else if (head == "kcache") *out = {m->kcache, kv};
    else if (head == "vcache") *out = {m->vcache, kv};
    else if (head == "rope") *out = {m->rope, (size_t)C.max_ctx * C.head_dim * 4};
    else if (head == "logits") *out = {m->logits, V * 4};
    else if (head == "token") *out = {m->token, 4};
    else if (head == "pos") *out = {m->pos, 4};
    else if (head == "hidden") *out = {m->h, D * 4};
    else if (head == "hidden_in") *out = {m->s, D * 4};
    else if (head == "hidden_norm") *out = {m->hn, D * 4};
    else if (head == "embed_scale") *out = {m->embed_scale, D * 4};
    else if (head == "history") *out = {m->hist, (size_t)(C.max_ctx + 1) * 4};
    else if (head.rfind("layer", 0) == 0) {
        int L = -1;
        try {
            L = std::stoi(head.substr(5));
        } catch (...) {
            return false;
        }
        if (L < 0 || L >= C.n_layers) return false;
        Layer& ly = m->layers[L];
        std::string w, part;
        split(rest, w, part);
        if (w == "attn_gain") *out = {ly.attn_gain, D * 2};
        else if (w == "ffn_gain") *out = {ly.ffn_gain, D * 2};
        else if (w == "wq") return matparts(ly.wq, part);
        else if (w == "wk") return matparts(ly.wk, part);
        else if (w == "wv") return matparts(ly.wv, part);
        else if (w == "wo") return matparts(ly.wo, part);
        else if (w == "w1") return matparts(ly.w1, part);
        else if (w == "w3") return matparts(ly.w3, part);
        else if (w == "w2") return matparts(ly.w2, part);
        else return false;
    } else return false;
    return true;
}

// tensor ids of the synthetic weights
static uint64_t tid_layer(int L, int k) { return 1000ull + 16ull * (uint64_t)L + (uint64_t)k; }
constexpr uint64_t kTidEmbed = 10, kTidFinalGain = 11, kTidLm = 12;

static int synth_mat(iam_model* m, Mat& w, uint64_t seed, uint64_t tid, uint16_t* scratch, size_t scratch_elems)
{
    Ctx* c = m->c;
    IAM_REQUIRE((size_t)w.out_dim * w.in_dim <= scratch_elems, "synthesize: matrix larger than its staging buffer");
    IAM_TRY(gen_f16(c, seed, tid, (size_t)w.out_dim * w.in_dim, 0.0, 0.02, scratch));
    IAM_TRY(zero_async(c, w.probes, (size_t)std::max(w.in_dim, kProbes) * 2));
    IAM_TRY(bucketize(c, scratch, w.out_dim, w.in_dim, w.buckets, w.stats, w.probes));
    IAM_TRY(iam_stats_compact(static_cast<iam_ctx*>(c), w.stats, (size_t)w.in_dim * 16, 4, 3, w.stats3));
    return IAM_OK;
}

}  // namespace iam

using namespace iam;

extern "C" {

int iam_model_create(iam_ctx* c, const iam_model_config* cfg, iam_model** out)
{
    if (!c || !cfg || !out) return fail(IAM_E_INVALID, "model_create: null argument");
    *out = nullptr;
    const iam_model_config& C = *cfg;
    IAM_REQUIRE(C.n_layers >= 1, "model: n_layers must be positive");
    IAM_REQUIRE(C.head_dim == 128, "model: head_dim must be 128");
    IAM_REQUIRE(C.n_heads * C.head_dim == C.dim, "model: dim must equal n_heads * head_dim");
    IAM_REQUIRE(C.n_kv_heads >= 1 && C.n_heads % C.n_kv_heads == 0 && C.n_heads / C.n_kv_heads <= 8,
                "model: n_heads must be a multiple of n_kv_heads (at most 8 per KV head)");
    IAM_REQUIRE(C.dim >= kProbes && C.dim % 1024 == 0 && C.dim <= 16384,
                "model: dim must be a multiple of 1024 in [4096, 16384] (the cutoff reads 4096 inputs)");
    IAM_REQUIRE(C.ffn_dim >= kProbes && C.ffn_dim % 16 == 0, "model: ffn_dim must be >= 4096 and a multiple of 16");
    IAM_REQUIRE(C.vocab >= 16 && C.vocab % 16 == 0, "model: vocab must be a positive multiple of 16");
    IAM_REQUIRE(C.max_ctx >= 1 && C.max_ctx <= 8192, "model: max_ctx must be in [1, 8192]");
    IAM_REQUIRE(C.dim / 256 <= kMaxChunks && C.ffn_dim / 256 < kMaxChunks, "model: dims too large");

    iam_model* m = new iam_model();
    m->c = c;
    m->cfg = C;
    m->layers.resize(C.n_layers);
    const int D = C.dim, F = C.ffn_dim, KVD = C.n_kv_heads * C.head_dim;
    int rc = IAM_OK;
    auto T = [&](int r) {
        if (rc == IAM_OK) rc = r;
    };
    for (int L = 0; L < C.n_layers && rc == IAM_OK; L++) {
        Layer& ly = m->layers[L];
        T(alloc_mat(m, ly.wq, D, D));
        T(alloc_mat(m, ly.wk, KVD, D));
        T(alloc_mat(m, ly.wv, KVD, D));
        T(alloc_mat(m, ly.wo, D, D));
        T(alloc_mat(m, ly.w1, F, D));
        T(alloc_mat(m, ly.w3, F, D));
        T(alloc_mat(m, ly.w2, D, F));
        T(alloc_t(m, D, &ly.attn_gain));
        T(alloc_t(m, D, &ly.ffn_gain));
    }
    T(alloc_mat(m, m->lm, C.vocab, D));
    T(alloc_t(m, (size_t)C.vocab * D, &m->embed));
    T(alloc_t(m, D, &m->final_gain));
    const size_t kv = (size_t)C.n_layers * C.max_ctx * KVD;
    T(alloc_t(m, kv, &m->kcache));
    T(alloc_t(m, kv, &m->vcache));
    T(alloc_t(m, (size_t)C.max_ctx * C.head_dim, &m->rope));
    T(alloc_t(m, D, &m->embed_scale));
    for (float** p : {&m->h, &m->hn, &m->q, &m->qr, &m->att, &m->o, &m->d}) T(alloc_t(m, D, p));
    T(alloc_t(m, KVD, &m->k));
    T(alloc_t(m, KVD, &m->v));
    for (float** p : {&m->g, &m->u, &m->s}) T(alloc_t(m, F, p));
    T(alloc_t(m, C.vocab, &m->logits));
    T(alloc_t(m, 1, &m->token));
    T(alloc_t(m, 1, &m->pos));
    T(alloc_t(m, C.max_ctx + 1, &m->hist));
    if (rc == IAM_OK) {
        std::vector<float> table((size_t)C.max_ctx * C.head_dim);
        rc = iam_rope_table(C.rope_theta, C.head_dim, C.max_ctx, table.data());
        if (rc == IAM_OK) rc = iam_write(c, m->rope, 0, table.data(), table.size() * 4);
    }
    if (rc == IAM_OK) rc = iam_model_reset_caches(m);
    if (rc != IAM_OK) {
        std::string err = iam_last_error();
        iam_model_destroy(m);
        return fail(rc, err);
    }
    *out = m;
    return IAM_OK;
}

int iam_model_destroy(iam_model* m)
{
    if (!m) return IAM_OK;
    (void)hipStreamSynchronize(m->c->stream);
    drop_graph(m);
    for (void* p : m->owned) (void)ctx_free(m->c, p);
    delete m;
    return IAM_OK;
}

int iam_model_synthesize(iam_model* m, uint64_t seed)
{
    if (!m) return fail(IAM_E_INVALID, "model_synthesize: null model");
    Ctx* c = m->c;
    const iam_model_config& C = m->cfg;
    // the largest matrix: dim x dim (wq, wo), ffn x dim (w1, w3, w2) or vocab x dim
    size_t maxw = (size_t)C.vocab * C.dim;
    maxw = std::max(maxw, (size_t)C.ffn_dim * C.dim);
    maxw = std::max(maxw, (size_t)C.dim * C.dim);
    uint16_t* scratch = nullptr;
    IAM_TRY(ctx_alloc(c, maxw * 2, (void**)&scratch));
    int rc = IAM_OK;
    for (int L = 0; L < C.n_layers && rc == IAM_OK; L++) {
        Layer& ly = m->layers[L];
        Mat* ws[7] = {&ly.wq, &ly.wk, &ly.wv, &ly.wo, &ly.w1, &ly.w3, &ly.w2};
        for (int k = 0; k < 7 && rc == IAM_OK; k++) rc = synth_mat(m, *ws[k], seed, tid_layer(L, k), scratch, maxw);
        if (rc == IAM_OK) rc = gen_f16(c, seed, tid_layer(L, 7), C.dim, 1.0, 0.01, ly.attn_gain);
        if (rc == IAM_OK) rc = gen_f16(c, seed, tid_layer(L, 8), C.dim, 1.0, 0.01, ly.ffn_gain);
    }
    if (rc == IAM_OK) rc = synth_mat(m, m->lm, seed, kTidLm, scratch, maxw);
    if (rc == IAM_OK) rc = gen_f16(c, seed, kTidEmbed, (size_t)C.vocab * C.dim, 0.0, 0.02, m->embed);
    if (rc == IAM_OK) rc = gen_f16(c, seed, kTidFinalGain, C.dim, 1.0, 0.01, m->final_gain);
    hipError_t e = hipStreamSynchronize(c->stream);
    int rc2 = ctx_free(c, scratch);
    if (rc != IAM_OK) return rc;
    if (e != hipSuccess) return fail(IAM_E_HIP, std::string("synthesize: ") + hipGetErrorString(e));
    return rc2;
}

int iam_model_reset_caches(iam_model* m)
{
    if (!m) return fail(IAM_E_INVALID, "reset_caches: null model");
    const iam_model_config& C = m->cfg;
    const size_t kv = (size_t)C.n_layers * C.max_ctx * C.n_kv_heads * C.head_dim * 2;
    IAM_TRY(zero_async(m->c, m->kcache, kv));
    IAM_TRY(zero_async(m->c, m->vcache, kv));
    IAM_TRY(zero_async(m->c, m->hist, (size_t)(C.max_ctx + 1) * 4));
    IAM_TRY(zero_async(m->c, m->pos, 4));
    IAM_TRY(zero_async(m->c, m->token, 4));
    IAM_CHECK_HIP(hipStreamSynchronize(m->c->stream));
    return IAM_OK;
}

int iam_model_forward(iam_model* m, int token, int pos, float effort, float* logits)
{
    if (!m || !logits) return fail(IAM_E_INVALID, "model_forward: null argument");
    const iam_model_config& C = m->cfg;
    IAM_REQUIRE(pos >= 0 && pos < C.max_ctx, "model_forward: pos outside the KV capacity");
    IAM_REQUIRE(token >= 0 && token < C.vocab, "model_forward: token outside the vocabulary");
    IAM_REQUIRE(!std::isnan(effort), "model_forward: effort is NaN");
    IAM_TRY(check_dev_range(m->c, logits, (size_t)C.vocab * 4, "model_forward logits"));
    IAM_TRY(reserve(m, effort));
    IAM_TRY(launch(m->c, "set_int", k_set_int, dim3(1), dim3(1), 0, m->token, token));
    IAM_TRY(launch(m->c, "set_int", k_set_int, dim3(1), dim3(1), 0, m->pos, pos));
    return step(m, effort, nullptr, logits, false);
}

int iam_model_step_device(iam_model* m, float effort, const float* hidden_override)
{
    if (!m) return fail(IAM_E_INVALID, "model_step: null model");
    IAM_REQUIRE(!std::isnan(effort), "model_step: effort is NaN");
    if (hidden_override) IAM_TRY(check_dev_range(m->c, hidden_override, (size_t)m->cfg.dim * 4, "model_step hidden"));
    IAM_TRY(reserve(m, effort));
    return step(m, effort, hidden_override, m->logits, true);
}

int iam_model_generate(iam_model* m, const int* prompt, int n_prompt, int n_new, float effort, int use_graph,
                       int* out_tokens)
{
    if (!m || (!prompt && n_prompt) || (!out_tokens && n_new)) return fail(IAM_E_INVALID, "generate: null argument");
    const iam_model_config& C = m->cfg;
    IAM_REQUIRE(n_prompt >= 1 && n_new >= 0, "generate: need at least one prompt token");
    IAM_REQUIRE(n_prompt + n_new <= C.max_ctx, "generate: prompt + new tokens exceed the KV capacity");
    IAM_REQUIRE(!std::isnan(effort), "generate: effort is NaN");
    for (int i = 0; i < n_prompt; i++)
        IAM_REQUIRE(prompt[i] >= 0 && prompt[i] < C.vocab, "generate: prompt token outside the vocabulary");
    Ctx* c = m->c;
    IAM_TRY(reserve(m, effort));
    IAM_TRY(launch(c, "set_int", k_set_int, dim3(1), dim3(1), 0, m->pos, 0));
    if (use_graph && (m->exec == nullptr || m->graph_effort != effort || m->graph_override ||
                      m->graph_gen != c->scratch_gen))
        IAM_TRY(capture_step(m, effort, false));
    auto one = [&]() -> int {
        if (use_graph) {
            IAM_CHECK_HIP(hipGraphLaunch(m->exec, c->stream));
            return IAM_OK;
        }
        return step(m, effort, nullptr, m->logits, true);
    };
    // prefill token by token through the decode path (test_generation.cpp:202-210)
    for (int i = 0; i < n_prompt; i++) {
        IAM_TRY(launch(c, "set_int", k_set_int, dim3(1), dim3(1), 0, m->token, prompt[i]));
        IAM_TRY(one());
    }
    // the pick of the last prompt step is the first new token; each further
    // step consumes the token the previous step picked
    for (int t = 1; t < n_new; t++) IAM_TRY(one());
    if (n_new > 0) {
        std::vector<int> hist(C.max_ctx + 1);
        IAM_CHECK_HIP(hipMemcpyAsync(hist.data(), m->hist, hist.size() * 4, hipMemcpyDeviceToHost, c->stream));
        IAM_CHECK_HIP(hipStreamSynchronize(c->stream));
        for (int t = 0; t < n_new; t++) out_tokens[t] = hist[n_prompt + t];
    }
    return IAM_OK;
}

int iam_model_decode(iam_model* m, int n_steps, float effort, int use_graph)
{
    if (!m) return fail(IAM_E_INVALID, "decode: null model");
    IAM_REQUIRE(n_steps >= 0, "decode: negative step count");
    IAM_REQUIRE(!std::isnan(effort), "decode: effort is NaN");
    Ctx* c = m->c;
    IAM_TRY(reserve(m, effort));
    if (use_graph && (m->exec == nullptr || m->graph_effort != effort || m->graph_override ||
                      m->graph_gen != c->scratch_gen))
        IAM_TRY(capture_step(m, effort, false));
    for (int t = 0; t < n_steps; t++) {
        if (use_graph) IAM_CHECK_HIP(hipGraphLaunch(m->exec, c->stream));
        else IAM_TRY(step(m, effort, nullptr, m->logits, true));
    }
    return IAM_OK;
}

int iam_model_tensor(iam_model* m, const char* name, void** dev, size_t* bytes)
{
    if (!m || !name || !dev || !bytes) return fail(IAM_E_INVALID, "model_tensor: null argument");
    TensorRef r{};
    if (!lookup(m, name, &r, nullptr)) return fail(IAM_E_INVALID, std::string("model_tensor: unknown ") + name);
    *dev = r.p;
    *bytes = r.bytes;
    return IAM_OK;
}

int iam_model_matrix(iam_model* m, const char* name, iam_bucket_matrix* out)
{
    if (!m || !name || !out) return fail(IAM_E_INVALID, "model_matrix: null argument");
    TensorRef r{};
    const Mat* w = nullptr;
    if (!lookup(m, name, &r, &w) || !w) return fail(IAM_E_INVALID, std::string("model_matrix: unknown ") + name);
    *out = w->desc();
    return IAM_OK;
}

int iam_model_set_embed_scale(iam_model* m, const float* scale_host)
{
    if (!m) return fail(IAM_E_INVALID, "set_embed_scale: null model");
    if (!scale_host) {
        m->use_scale = false;
    } else {
        IAM_TRY(iam_write(m->c, m->embed_scale, 0, scale_host, (size_t)m->cfg.dim * 4));
        m->use_scale = true;
    }
    return drop_graph(m);   // the captured step depends on it
}

}  // extern "C"
