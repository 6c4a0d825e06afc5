/*
 * CPU oracle for the input-adaptive sparse decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this code.  It is used by tests/, by __graft_entry__.smoke() as the
 * checker, and by bench.py's cpu_baseline leg as the timed CPU port.
 *
 * Every function restates the reference algorithm in plain C with IEEE fp32
 * semantics (built with -ffp-contract=off, no fast-math) and cites the
 * reference file:line it follows.  How each function is pinned (golden
 * vectors, known-answer tests, closed forms, brute force) is listed in the
 * header of oracle.c.
 */
#ifndef IAM_ORACLE_H
#define IAM_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_PROBES_COUNT 4096        /* bucketMul.cl:18 */
#define ORC_CUTOFF_SCALE 100000.0f   /* bucketMul.cl:17 */
#define ORC_MAX_ROUNDS 20            /* bucketMul.cl:148 */

/* ---- fp16 helpers -------------------------------------------------------- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);                 /* round to nearest even */
uint16_t orc_f64_to_f16(double d);                /* round to nearest even, one rounding */
void orc_f64_to_f16_n(const double* in, uint16_t* out, size_t n);
void orc_f32_to_f16_n(const float* in, uint16_t* out, size_t n);
void orc_f16_to_f32_n(const uint16_t* in, float* out, size_t n);
/* preprocess_layer_fixed_gpu.py:40-89 pack/unpack of a value with a 4-bit position */
uint16_t orc_pack_fp16(float value, int position);
void orc_unpack_fp16(uint16_t packed, float* value, int* position);

/* ---- synthetic data (shared definition with the GPU generator) ---------- */
/* Counter-based: element n of tensor `tensor_id` for seed `seed`.
 * normal = (sum of 12 uniform uint32 - 6*2^32) / 2^32 (Irwin-Hall, var 1).
 * The f16 variant rounds mean + sigma*normal (double) once to fp16; the f32
 * variant rounds it once to float. */
double orc_gen_normal(uint64_t seed, uint64_t tensor_id, uint64_t n);
uint32_t orc_gen_u32(uint64_t seed, uint64_t tensor_id, uint64_t n);
void orc_gen_f16(uint64_t seed, uint64_t tensor_id, size_t count, double mean, double sigma, uint16_t* out);
void orc_gen_f32(uint64_t seed, uint64_t tensor_id, size_t count, double mean, double sigma, float* out);
void orc_gen_tokens(uint64_t seed, uint64_t tensor_id, size_t count, uint32_t vocab, int32_t* out);

/* ---- bucket layout producer (preprocess_layer_fixed_gpu.py:110-242) ----- */
/* W: fp16 [out_dim][in_dim] row-major.  Outputs: buckets [16*in][out/16],
 * stats [16*in][4], probes [in].  Returns 0, or -1 if out_dim % 16 != 0. */
int orc_bucketize(const uint16_t* W, int out_dim, int in_dim,
                  uint16_t* buckets, uint16_t* stats, uint16_t* probes);
/* numpy float32 pairwise summation (the order np.mean uses on a contiguous axis) */
float orc_np_pairwise_sum_f32(const float* a, ptrdiff_t n);

/* ---- cutoff search (bucketMul.cl:68-214) --------------------------------- */
int orc_effort_quantile(float effort);            /* bucket_mul.hpp:164 */

typedef struct {
    int rounds;                 /* rounds executed (1..20) */
    int converged;              /* 1 = stopped on a convergence test, 0 = ran out of rounds */
    float init_min, init_max;
    float bounds[ORC_MAX_ROUNDS];   /* bound tested in each round */
    int counts[ORC_MAX_ROUNDS];     /* #(imp > bound) in each round */
    float final_min, final_max;
    int final_min_count, final_max_count;
} orc_cutoff_trace;

/* importance, bucketMul.cl:101-117 (4096 values; probes offset expNo*4096) */
void orc_importance(const float* x, const uint16_t* probes, int exp_no, float* imp);
/* returns the cutoff exactly as the reference kernel writes it */
float orc_find_cutoff(const float* x, const uint16_t* probes, int exp_no, int quantile,
                      orc_cutoff_trace* trace);
/* same search on a precomputed importance array of 4096 values */
float orc_find_cutoff_imp(const float* imp, int quantile, orc_cutoff_trace* trace);

/* ---- row selection (bucketMul.cl:351-386) -------------------------------- */
/* stats: [n_rows_total][stats_channels], channel 3 used.  Writes mask[expert_rows]
 * (1 = selected) for rows of expert exp_no; returns the selected count. */
int64_t orc_select_rows(const float* x, const uint16_t* stats, int stats_channels,
                        int exp_no, int expert_rows, int in_size, float cutoff,
                        uint8_t* mask);
/* block-structured selection: rank k of every input of a block of `block`
 * consecutive inputs when rank k of any of them passes (block 1: the above) */
int64_t orc_select_rows_block(const float* x, const uint16_t* stats, int stats_channels,
                              int exp_no, int expert_rows, int in_size, float cutoff, int block,
                              uint8_t* mask);

/* ---- bucket walk + integrate (bucketMul.cl:392-497) ---------------------- */
/* y[out_dim = 16*C] = sum over selected rows r (mask) of x[r/16]*W[r][c] at
 * y[c*16 + (bits & 15)].  acc64 != 0: fp64 accumulation (reference value);
 * otherwise fp32 in row order.  y is overwritten. */
void orc_bucket_walk(const uint16_t* buckets, int bucket_cols, int exp_no, int expert_rows,
                     const uint8_t* mask, const float* x, float* y, int acc64);

/* calcDispatch + mul in one call (bucket_mul.hpp:254-267).  Returns S. */
int64_t orc_bucketmul(const float* x, const uint16_t* stats, const uint16_t* probes,
                      const uint16_t* buckets, int exp_no, int in_size, int bucket_cols,
                      int expert_rows, float effort, float* y, float* cutoff_out,
                      uint8_t* mask_out, int acc64);

/* ---- layer kernels -------------------------------------------------------- */
/* rmsNorm32fast (aux.cl:156-196) followed by the fp16 gain (aux.cl:434-440) */
void orc_rmsnorm_gain(const float* in, const uint16_t* gain, int n, float eps, float* out);
/* silu32 (matrix.cl:27-32): out = x3*x1/(1+exp(-x1)) */
void orc_silu_mul(const float* x1, const float* x3, int n, float* out);
/* precompute_rope_cache (attention.hpp:207-235): table[pos][64][2] = cos,sin */
void orc_rope_table(double theta, int head_dim, int max_pos, float* table);
/* rope_mx (aux.cl:227-248) over n_heads heads of head_dim with table row for pos */
void orc_rope(const float* in, const float* table_row, int n_heads, int head_dim, float* out);
/* fetchRow16to32 (aux.cl:442-452) */
void orc_embed(const uint16_t* table, int cols, int token, float* out);
/* add32 (bucketMul.cl:517-520) */
void orc_add(const float* a, const float* b, int n, float* out);
/* decode attention (aux.cl:370-540; attention.hpp:311-404) over an fp16 GQA
 * cache K,V [ctx_cap][n_kv][hd] for positions 0..n_tok-1.  fp64 evaluation,
 * exp(s) with no maximum subtracted (as the reference). */
void orc_attention_f16kv(const float* q, const uint16_t* kcache, const uint16_t* vcache,
                         int n_tok, int n_heads, int n_kv, int head_dim, float* out);
/* the reference's fp32 attention over its repeated-head cache layout
 * K, V [ctx_cap][n_heads][head_dim] fp32 (model.hpp:97-98) for positions
 * 0..n_tok-1, in the fixed order of splits of ORC_ATT32_SPLIT positions */
#define ORC_ATT32_SPLIT 64
void orc_attention_f32rep(const float* q, const float* kcache, const float* vcache, int n_tok,
                          int n_heads, int head_dim, float* out);
/* RoPE of q and k, and the K/V rows of one position repeated to n_heads heads
 * (attention.hpp:172-189, :281-309); k_row and v_row are [n_heads][head_dim] */
void orc_rope_kv_rep32(const float* q, const float* k, const float* v, const float* table_row,
                       int n_heads, int n_kv, int head_dim, float* q_out, float* k_row, float* v_row);
/* matmul16x32 (aux.cl:454-490) with 256 work-items per row (model.hpp:207-227) */
#define ORC_DENSE_WG 256
void orc_matmul_f16_dense(const uint16_t* W, const float* x, int rows, int cols, float* out);
/* argmax, first maximum (test_generation.cpp:235, 276) */
int orc_argmax(const float* v, int n);

/* ---- model (model.hpp:152-231, transformer_layer.hpp:75-122) ------------ */
typedef struct {
    int n_layers, dim, ffn_dim, n_heads, n_kv_heads, head_dim, vocab, max_ctx;
    double rope_theta;
    float norm_eps;
} orc_model_config;

typedef struct {
    const uint16_t *buckets, *stats, *probes;
    int in_dim, out_dim;        /* bucket_cols = out_dim/16, rows = 16*in_dim */
} orc_matrix;

typedef struct {
    orc_matrix wq, wk, wv, wo, w1, w3, w2;
    const uint16_t *attn_gain, *ffn_gain;
} orc_layer;

typedef struct {
    orc_model_config cfg;
    const orc_layer* layers;
    const uint16_t* embed;      /* [vocab][dim] */
    const uint16_t* final_gain; /* [dim] */
    orc_matrix lm_head;         /* bucket layout */
    uint16_t *kcache, *vcache;  /* [n_layers][max_ctx][n_kv][hd] fp16 */
    float* rope;                /* [max_ctx][64][2] */
    const uint16_t* lm_dense;   /* [vocab][dim] fp16: when set, the reference's dense
                                   head (matmul16x32) instead of lm_head */
} orc_model;

/* one decode step; writes logits[vocab]; the KV cache at pos is written.
 * hidden_in != NULL replaces the embedding lookup (for skew experiments). */
void orc_layer_forward(const orc_model* m, int layer, int pos, float effort, float* h);
void orc_model_forward(const orc_model* m, int token, int pos, float effort,
                       const float* hidden_in, float* logits);

/* selection of orc_bucketmul and the forwards above: blocks of `block`
 * inputs (orc_select_rows_block) for efforts below below_effort; block 1
 * (the default) is the reference's per-row selection */
void orc_set_selection_block(int block, float below_effort);

/* threads the OpenMP loops use (1 when built without OpenMP) */
int orc_threads(void);

#ifdef __cplusplus
}
#endif
#endif
