// Mistral-shaped decoder over the bucket-layout weights.
//
// MistralModel::forward (model.hpp:152-231) = embedding gather, 32 x
// TransformerLayer::forward (transformer_layer.hpp:75-122: norm -> attention
// -> +res -> norm -> FFN -> +res), final norm, LM head, greedy argmax
// (test_generation.cpp:235/276).  A decode step is 5 launches per layer and
// one for the LM head:
//   q/k/v walk  (input: residual add of the previous FFN + attention norm;
//                the first layer gathers the embedding row instead)
//   attention   (RoPE of q and k and the fp16 KV append in its prologue)
//   o walk      (input: the attention output o / l)
//   w1/w3 walk  (input: residual add of o + FFN norm; its tiles' last
//                workgroups store the SiLU gate)
//   w2 walk     (input: the gate)
//   LM head walk (input: residual add + final norm; its last workgroup picks
//                the next token and advances the position)
// Each walk flushes its sums into fp64 accumulators with atomics; the next
// launch reads them, and a later launch clears them (see step()).  The
// position and token live in device memory, so a whole step is captured
// once as a HIP graph and replayed per token with no host round trip.
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

// a captured run of decode steps at one effort
struct StepGraph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    float effort = -1.0f;
    uint64_t gen = 0;   // Ctx::scratch_gen at capture
};
constexpr int kGraphSteps = 8;

}  // namespace iam

struct iam_model {
    iam_ctx* c = nullptr;
    iam_model_config cfg{};
    std::vector<iam::Layer> layers;
    uint16_t* embed = nullptr;
    uint16_t* final_gain = nullptr;
    iam::Mat lm;
    // the reference's dense fp16 LM head [vocab][dim] (caller-owned), used
    // instead of the bucket-layout one when set
    const uint16_t* lm_dense = nullptr;
    uint16_t* kcache = nullptr;
    uint16_t* vcache = nullptr;
    float* rope = nullptr;
    float* embed_scale = nullptr;   // optional per-channel scale of the gathered embedding
    bool use_scale = false;
    // residual stream: ha[L] enters layer L, hb[L] enters its FFN block
    float* ha = nullptr;
    float* hb = nullptr;
    float* hidden = nullptr;        // after the last layer
    float* hn = nullptr;            // the last normalized input (the LM head's, after a step)
    float* att_x = nullptr;         // the attention output o / l of the last layer
    float* s = nullptr;             // SiLU gate output [ffn]
    float* hidden_in = nullptr;     // embedding override staging
    // accumulators (8 bytes per value): q|k|v, attention o|l, o, gate, up,
    // down, logits; zero between steps
    void* att_part = nullptr;       // attention: the splits' partial sums
    uint32_t* att_ctr = nullptr;    // attention: arrival counters per query head
    void *acc_qkv = nullptr, *acc_att = nullptr, *acc_o = nullptr, *acc_g = nullptr, *acc_u = nullptr,
         *acc_d = nullptr, *acc_lm = nullptr;
    uint32_t* tile_ctr = nullptr;   // gate/up tiles, then LM head tiles, then the pick counter
    uint2* cand = nullptr;          // LM head tile maxima
    float* cut = nullptr;           // cutoffs of the last group [3]
    // the cutoff searches' hints, each matrix's cutoff of the previous step:
    // per layer q, k, v, o, w1, w3, w2 (8 slots), then the LM head
    float* hints = nullptr;
    uint32_t* slice_counts = nullptr;   // [3][slice_cap]
    int slice_cap = 0;
    float* logits = nullptr;
    int* token = nullptr;
    int* pos = nullptr;
    int* hist = nullptr;            // token history [max_ctx + 1]
    int host_pos = 0;               // the position the next step computes
    // captured decode steps: one step, and kGraphSteps consecutive ones (the
    // decode loops launch the latter while that many remain, so the gap
    // between two graph launches comes once per kGraphSteps steps)
    iam::StepGraph one, multi;
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

static size_t acc_bytes(size_t n) { return n * 8; }

static WalkMat walk_mat(iam_model* m, const Mat& w, int slot, int in_size, void* acc)
{
    WalkMat wm{};
    wm.mat = w.desc();
    wm.in_size = in_size;
    wm.cutoff = m->cut + slot;
    wm.slice_count = m->slice_counts + (size_t)slot * m->slice_cap;
    wm.acc = acc;
    return wm;
}

// One decode step reading token/pos from device memory; logits_out is the
// model's own buffer or a caller buffer of vocab floats.  With pick, the LM
// head's last workgroup writes the next token, the history and pos + 1.
//
// Accumulators: each is written by one launch and read by the next one(s);
// the launch after its last reader clears it, so all are zero between steps:
//   qkv  written by the q/k/v walk, read by attention, cleared by the o walk
//   att  written by attention, read by the o walk, cleared by the w1/w3 walk
//   o    written by the o walk, read by the w1/w3 walk, cleared by the w2 walk
//   gate/up  written by the w1/w3 walk, taken (read and cleared) by its own
//        tiles' last workgroups
//   down written by the w2 walk, read by the next q/k/v walk (or the LM
//        head), cleared by the next attention (or the LM head's last
//        workgroup)
//   logits   taken by the LM head's tiles' last workgroups
// Models wider than 4096 (the walk normalises 4096 inputs itself) run the
// residual add + norm as a kernel of its own before the walk.
static int step(iam_model* m, float effort, const float* hidden_override, float* logits_out, bool pick)
{
    Ctx* c = m->c;
    const iam_model_config& C = m->cfg;
    const int D = C.dim, F = C.ffn_dim, KVD = C.n_kv_heads * C.head_dim;
    const bool wide = D != kProbes;
    const size_t kv_layer = (size_t)C.max_ctx * KVD;
    char* qkv = static_cast<char*>(m->acc_qkv);
    const int T13 = walk_tiles(F / 16);
    for (int L = 0; L < C.n_layers; L++) {
        Layer& ly = m->layers[L];
        uint16_t* kc = m->kcache + (size_t)L * kv_layer;
        uint16_t* vc = m->vcache + (size_t)L * kv_layer;
        float* ha = m->ha + (size_t)L * D;
        float* hb = m->hb + (size_t)L * D;
        const float* hprev = L == 0 ? nullptr : m->hb + (size_t)(L - 1) * D;
        // ---- q, k, v (attention.hpp:160-170) with the attention norm
        // (transformer_layer.hpp:96-100) and the previous FFN's residual
        {
            WalkGroup g;
            g.label = IAM_WALK_GROUP_QKV;
            g.n = 3;
            g.m[0] = walk_mat(m, ly.wq, 0, D, qkv);
            g.m[1] = walk_mat(m, ly.wk, 1, D, qkv + acc_bytes(D));
            g.m[2] = walk_mat(m, ly.wv, 2, D, qkv + acc_bytes(D + KVD));
            for (int j = 0; j < 3; j++) g.m[j].hint = m->hints + (size_t)L * 8 + j;
            // k and v: one column tile each, so every slice adds into the
            // same outputs; the odd slices use second copies (after v),
            // which attention adds
            g.m[1].acc2 = qkv + acc_bytes(D + 2 * KVD);
            g.m[2].acc2 = qkv + acc_bytes(D + 3 * KVD);
            g.effort = effort;
            g.gain = ly.attn_gain;
            g.eps = C.norm_eps;
            if (!wide) {
                for (int i = 0; i < 3; i++) g.m[i].x = m->hn;
                if (L > 0) {
                    g.in_mode = kInResNorm;
                    g.h = hprev;
                    g.res_acc = m->acc_d;
                } else if (hidden_override) {
                    g.in_mode = kInResNorm;
                    g.h = hidden_override;
                } else {
                    g.in_mode = kInEmbedNorm;
                    g.embed = m->embed;
                    g.token = m->token;
                    g.embed_scale = m->use_scale ? m->embed_scale : nullptr;
                    g.vocab = C.vocab;
                }
                g.h_out = ha;
            } else {
                if (L > 0) {
                    IAM_TRY(resnorm(c, hprev, m->acc_d, ha, ly.attn_gain, D, C.norm_eps, m->hn));
                } else {
                    if (hidden_override) {
                        IAM_TRY(launch(c, "copy_hidden", k_copy_f32, dim3((D + 255) / 256), dim3(256), 0,
                                       hidden_override, ha, D));
                    } else {
                        IAM_TRY(embed(c, m->embed, D, C.vocab, m->token, ha));
                        if (m->use_scale)
                            IAM_TRY(launch(c, "embed_scale", k_scale_vec, dim3((D + 255) / 256), dim3(256), 0, ha,
                                           (const float*)m->embed_scale, D));
                    }
                    IAM_TRY(resnorm(c, ha, nullptr, nullptr, ly.attn_gain, D, C.norm_eps, m->hn));
                }
                for (int i = 0; i < 3; i++) g.m[i].x = m->hn;
                g.in_mode = kInX;
            }
            IAM_TRY(walk_group(c, g));
        }
        // ---- attention (attention.hpp:172-200): RoPE, KV append, split
        // attention into o|l; clears the previous FFN's down accumulator
        {
            AttnLaunch A{};
            A.qkv_acc = m->acc_qkv;
            A.kv_copies = 2;
            A.rope = m->rope;
            A.kc = kc;
            A.vc = vc;
            A.pos = m->pos;
            A.n_heads = C.n_heads;
            A.n_kv = C.n_kv_heads;
            A.max_ctx = C.max_ctx;
            A.acc = m->acc_att;
            A.part = m->att_part;
            A.head_ctr = m->att_ctr;
            A.zero_p = m->acc_d;
            A.zero_n = D;
            A.atomic_splits = kAttnAtomicSplits;
            IAM_TRY(attention_launch(c, A));
        }
        // ---- o projection (attention.hpp:198-200)
        {
            WalkGroup g;
            g.label = IAM_WALK_GROUP_O;
            g.n = 1;
            g.m[0] = walk_mat(m, ly.wo, 0, D, m->acc_o);
            g.m[0].hint = m->hints + (size_t)L * 8 + 3;
            g.m[0].x = m->att_x;
            g.effort = effort;
            g.in_mode = kInAttn;
            g.attn_acc = m->acc_att;
            g.zero_p[0] = m->acc_qkv;
            g.zero_n[0] = D + 4 * KVD;
            IAM_TRY(walk_group(c, g));
        }
        // ---- gate and up (feedforward.hpp:60-78) with the residual add of o
        // and the FFN norm (transformer_layer.hpp:104-112); SiLU gate
        {
            WalkGroup g;
            g.label = IAM_WALK_GROUP_FFN13;
            g.n = 2;
            g.m[0] = walk_mat(m, ly.w1, 0, D, m->acc_g);
            g.m[1] = walk_mat(m, ly.w3, 1, D, m->acc_u);
            g.m[0].hint = m->hints + (size_t)L * 8 + 4;
            g.m[1].hint = m->hints + (size_t)L * 8 + 5;
            g.m[0].tile_ctr = g.m[1].tile_ctr = m->tile_ctr;
            g.effort = effort;
            g.gain = ly.ffn_gain;
            g.eps = C.norm_eps;
            if (!wide) {
                g.in_mode = kInResNorm;
                g.h = ha;
                g.res_acc = m->acc_o;
                g.h_out = hb;
                g.m[0].x = g.m[1].x = m->hn;
            } else {
                IAM_TRY(resnorm(c, ha, m->acc_o, hb, ly.ffn_gain, D, C.norm_eps, m->hn));
                g.in_mode = kInX;
                g.m[0].x = g.m[1].x = m->hn;
            }
            g.fin = kFinSilu;
            g.silu_out = m->s;
            // the attention sums, read by the o walk: zero for the next layer's adds
            g.zero_p[0] = m->acc_att;
            g.zero_n[0] = (int)attention_acc_words(C.n_heads);
            IAM_TRY(walk_group(c, g));
        }
        // ---- down (feedforward.hpp:82-84)
        {
            WalkGroup g;
            g.label = IAM_WALK_GROUP_FFN2;
            g.n = 1;
            g.m[0] = walk_mat(m, ly.w2, 0, F, m->acc_d);
            g.m[0].hint = m->hints + (size_t)L * 8 + 6;
            g.m[0].x = m->s;
            g.effort = effort;
            g.in_mode = kInX;
            g.zero_p[0] = m->acc_o;
            g.zero_n[0] = D;
            IAM_TRY(walk_group(c, g));
        }
    }
    // ---- final norm + the reference's dense LM head (model.hpp:181-227,
    // matmul16x32) + greedy pick
    if (m->lm_dense) {
        const float* hlast = m->hb + (size_t)(C.n_layers - 1) * D;
        IAM_TRY(resnorm(c, hlast, m->acc_d, m->hidden, m->final_gain, D, C.norm_eps, m->hn));
        IAM_TRY(matmul_f16_dense(c, m->lm_dense, m->hn, C.vocab, D, logits_out));
        if (pick) IAM_TRY(argmax(c, logits_out, C.vocab, m->token, m->pos, m->hist, C.max_ctx + 1));
        IAM_TRY(zero_async(c, m->acc_d, acc_bytes(D)));
        return IAM_OK;
    }
    // ---- final norm + LM head (model.hpp:181-227) + greedy pick
    {
        const float* hlast = m->hb + (size_t)(C.n_layers - 1) * D;
        WalkGroup g;
        g.label = IAM_WALK_GROUP_LM;
        g.n = 1;
        g.m[0] = walk_mat(m, m->lm, 0, D, m->acc_lm);
        g.m[0].hint = m->hints + (size_t)C.n_layers * 8;
        g.m[0].tile_ctr = m->tile_ctr + T13;
        g.m[0].y = logits_out;
        g.m[0].x = m->hn;
        g.effort = effort;
        g.gain = m->final_gain;
        g.eps = C.norm_eps;
        if (!wide) {
            g.in_mode = kInResNorm;
            g.h = hlast;
            g.res_acc = m->acc_d;
            g.h_out = m->hidden;
        } else {
            IAM_TRY(resnorm(c, hlast, m->acc_d, m->hidden, m->final_gain, D, C.norm_eps, m->hn));
            g.in_mode = kInX;
        }
        g.fin = kFinStore;
        const int Tlm = walk_tiles(C.vocab / 16);
        g.pick_ctr = m->tile_ctr + T13 + Tlm;
        g.tile_cand = m->cand;
        if (pick) {
            g.token_out = m->token;
            g.pos = m->pos;
            g.hist = m->hist;
            g.hist_len = C.max_ctx + 1;
        }
        g.final_zero = m->acc_d;
        g.final_zero_n = D;
        IAM_TRY(walk_group(c, g));
    }
    (void)T13;
    return IAM_OK;
}

static void drop_one(StepGraph& G)
{
    if (G.exec) (void)hipGraphExecDestroy(G.exec);
    if (G.graph) (void)hipGraphDestroy(G.graph);
    G = StepGraph{};
}

static int drop_graph(iam_model* m)
{
    drop_one(m->one);
    drop_one(m->multi);
    return IAM_OK;
}

// The captured graph of `steps` consecutive decode steps (1 or kGraphSteps)
// at this effort, captured where it is missing or stale (another effort, or
// a context scratch buffer reallocated since: the graph holds addresses).
static int step_graph(iam_model* m, float effort, int steps, hipGraphExec_t* out)
{
    Ctx* c = m->c;
    StepGraph& G = steps == 1 ? m->one : m->multi;
    if (G.exec && (G.effort != effort || G.gen != c->scratch_gen)) drop_one(G);
    if (!G.exec) {
        IAM_CHECK_HIP(hipStreamSynchronize(c->stream));
        IAM_CHECK_HIP(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
        c->capturing = true;
        int rc = IAM_OK;
        for (int s = 0; s < steps && rc == IAM_OK; s++) rc = step(m, effort, nullptr, m->logits, true);
        c->capturing = false;
        hipGraph_t g = nullptr;
        hipError_t e = hipStreamEndCapture(c->stream, &g);
        if (rc != IAM_OK) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        if (e != hipSuccess) return fail(IAM_E_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(e));
        G.graph = g;
        IAM_CHECK_HIP(hipGraphInstantiate(&G.exec, g, nullptr, nullptr, 0));
        G.effort = effort;
        G.gen = c->scratch_gen;
    }
    *out = G.exec;
    return IAM_OK;
}

// n decode steps from the device's token and position: graph launches of
// kGraphSteps steps while that many remain, then single steps.  Both graphs
// are made current before the first launch (a capture records and
// instantiates, it runs nothing), so a later call with more steps finds its
// graph ready.
static int run_steps(iam_model* m, int n, float effort, bool use_graph)
{
    if (!use_graph) {
        for (int t = 0; t < n; t++) IAM_TRY(step(m, effort, nullptr, m->logits, true));
        return IAM_OK;
    }
    if (n == 0) return IAM_OK;
    hipGraphExec_t x1 = nullptr, xk = nullptr;
    IAM_TRY(step_graph(m, effort, 1, &x1));
    IAM_TRY(step_graph(m, effort, kGraphSteps, &xk));
    for (int t = 0; t < n;) {
        const bool many = n - t >= kGraphSteps;
        IAM_CHECK_HIP(hipGraphLaunch(many ? xk : x1, m->c->stream));
        t += many ? kGraphSteps : 1;
    }
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
    else if (head == "hidden") *out = {m->hidden, D * 4};
    else if (head == "hidden_in") *out = {m->hidden_in, D * 4};
    else if (head == "hidden_norm") *out = {m->hn, D * 4};
    else if (head == "attention_out") *out = {m->att_x, D * 4};
    else if (head == "ffn_act") *out = {m->s, (size_t)C.ffn_dim * 4};
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
        else if (w == "h_in") *out = {m->ha + (size_t)L * D, D * 4};
        else if (w == "h_mid") *out = {m->hb + (size_t)L * D, D * 4};
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
    T(alloc_t(m, (size_t)C.n_layers * D, &m->ha));
    T(alloc_t(m, (size_t)C.n_layers * D, &m->hb));
    for (float** p : {&m->hidden, &m->hn, &m->att_x, &m->hidden_in}) T(alloc_t(m, D, p));
    T(alloc_t(m, F, &m->s));
    T(alloc_owned(m, acc_bytes(D + 4 * KVD), &m->acc_qkv));   // q | k | v | k, v of the odd slices
    T(alloc_owned(m, acc_bytes(attention_acc_words(C.n_heads)), &m->acc_att));
    T(alloc_owned(m, acc_bytes(attention_part_words(C.n_heads, C.n_kv_heads, C.max_ctx)), &m->att_part));
    T(alloc_t(m, (size_t)C.n_heads, &m->att_ctr));
    T(alloc_owned(m, acc_bytes(D), &m->acc_o));
    T(alloc_owned(m, acc_bytes(F), &m->acc_g));
    T(alloc_owned(m, acc_bytes(F), &m->acc_u));
    T(alloc_owned(m, acc_bytes(D), &m->acc_d));
    T(alloc_owned(m, acc_bytes(C.vocab), &m->acc_lm));
    const int T13 = walk_tiles(F / 16), Tlm = walk_tiles(C.vocab / 16);
    T(alloc_t(m, (size_t)T13 + Tlm + 1, &m->tile_ctr));
    T(alloc_t(m, (size_t)Tlm, &m->cand));
    T(alloc_t(m, 3, &m->cut));
    T(alloc_t(m, (size_t)C.n_layers * 8 + 1, &m->hints));
    m->slice_cap = std::max(D, F);   // a slice holds at least one input
    T(alloc_t(m, (size_t)3 * m->slice_cap, &m->slice_counts));
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
    // the accumulators and counters are zero between steps; clear them
    // anyway, so that a reset also recovers from an interrupted step
    const int D = C.dim, F = C.ffn_dim, KVD = C.n_kv_heads * C.head_dim;
    IAM_TRY(zero_async(m->c, m->acc_qkv, acc_bytes(D + 4 * KVD)));
    IAM_TRY(zero_async(m->c, m->acc_att, acc_bytes(attention_acc_words(C.n_heads))));
    for (void* p : {m->acc_o, m->acc_d}) IAM_TRY(zero_async(m->c, p, acc_bytes(D)));
    for (void* p : {m->acc_g, m->acc_u}) IAM_TRY(zero_async(m->c, p, acc_bytes(F)));
    IAM_TRY(zero_async(m->c, m->acc_lm, acc_bytes(C.vocab)));
    const int T13 = walk_tiles(F / 16), Tlm = walk_tiles(C.vocab / 16);
    IAM_TRY(zero_async(m->c, m->tile_ctr, ((size_t)T13 + Tlm + 1) * 4));
    IAM_TRY(zero_async(m->c, m->att_ctr, (size_t)C.n_heads * 4));
    // a new sequence starts without hints (0: the full search)
    IAM_TRY(zero_async(m->c, m->hints, ((size_t)C.n_layers * 8 + 1) * 4));
    IAM_CHECK_HIP(hipStreamSynchronize(m->c->stream));
    m->host_pos = 0;
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
    IAM_REQUIRE(((uintptr_t)logits & 15) == 0, "model_forward: logits must be 16-byte aligned");
    IAM_TRY(launch(m->c, "set_int", k_set_int, dim3(1), dim3(1), 0, m->token, token));
    IAM_TRY(launch(m->c, "set_int", k_set_int, dim3(1), dim3(1), 0, m->pos, pos));
    m->host_pos = pos;   // forward does not advance the position
    return step(m, effort, nullptr, logits, false);
}

int iam_model_step_device(iam_model* m, float effort, const float* hidden_override)
{
    if (!m) return fail(IAM_E_INVALID, "model_step: null model");
    IAM_REQUIRE(!std::isnan(effort), "model_step: effort is NaN");
    if (hidden_override) {
        IAM_TRY(check_dev_range(m->c, hidden_override, (size_t)m->cfg.dim * 4, "model_step hidden"));
        IAM_REQUIRE(((uintptr_t)hidden_override & 15) == 0, "model_step: hidden must be 16-byte aligned");
    }
    IAM_REQUIRE(m->host_pos >= 0 && m->host_pos < m->cfg.max_ctx,
                "model_step: the position has reached the KV capacity");
    IAM_TRY(step(m, effort, hidden_override, m->logits, true));
    m->host_pos++;
    return IAM_OK;
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
    IAM_TRY(launch(c, "set_int", k_set_int, dim3(1), dim3(1), 0, m->pos, 0));
    m->host_pos = 0;
    // prefill token by token through the decode path (test_generation.cpp:202-210)
    for (int i = 0; i < n_prompt; i++) {
        IAM_TRY(launch(c, "set_int", k_set_int, dim3(1), dim3(1), 0, m->token, prompt[i]));
        IAM_TRY(run_steps(m, 1, effort, use_graph));
    }
    // the pick of the last prompt step is the first new token; each further
    // step consumes the token the previous step picked
    if (n_new > 1) IAM_TRY(run_steps(m, n_new - 1, effort, use_graph));
    m->host_pos = n_prompt + std::max(n_new - 1, 0);
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
    // positions host_pos .. host_pos + n_steps - 1 must fit the KV cache
    IAM_REQUIRE(m->host_pos >= 0 && (int64_t)m->host_pos + n_steps <= m->cfg.max_ctx,
                "decode: the steps would pass the KV capacity");
    IAM_TRY(run_steps(m, n_steps, effort, use_graph != 0));
    m->host_pos += n_steps;
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

int iam_model_set_position(iam_model* m, int pos)
{
    if (!m) return fail(IAM_E_INVALID, "set_position: null model");
    IAM_REQUIRE(pos >= 0 && pos <= m->cfg.max_ctx, "set_position: pos outside [0, max_ctx]");
    IAM_TRY(launch(m->c, "set_int", k_set_int, dim3(1), dim3(1), 0, m->pos, pos));
    m->host_pos = pos;
    return IAM_OK;
}

int iam_model_set_lm_dense(iam_model* m, const uint16_t* lm_dense)
{
    if (!m) return fail(IAM_E_INVALID, "set_lm_dense: null model");
    if (lm_dense) {
        IAM_TRY(check_dev_range(m->c, lm_dense, (size_t)m->cfg.vocab * m->cfg.dim * 2, "set_lm_dense matrix"));
        IAM_REQUIRE(((uintptr_t)lm_dense & 7) == 0, "set_lm_dense: the matrix must be 8-byte aligned");
    }
    m->lm_dense = lm_dense;
    return drop_graph(m);   // the captured step depends on it
}

int iam_model_set_embed_scale(iam_model* m, const float* scale_host)
{
    if (!m) return fail(IAM_E_INVALID, "set_embed_scale: null model");
    const bool was = m->use_scale;
    if (!scale_host) {
        m->use_scale = false;
    } else {
        IAM_TRY(iam_write(m->c, m->embed_scale, 0, scale_host, (size_t)m->cfg.dim * 4));
        m->use_scale = true;
    }
    // the captured steps read the scale buffer (or none): new contents need
    // no new capture, switching it on or off does
    return was != m->use_scale ? drop_graph(m) : IAM_OK;
}

}  // extern "C"
