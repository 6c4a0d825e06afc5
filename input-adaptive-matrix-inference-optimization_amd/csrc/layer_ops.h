// Host-side launchers of the layer kernels (no argument checks: the C ABI
// entry points and the model check shapes and ranges before calling them).
#pragma once

#include "internal.h"

namespace iam {

// rope_mx (aux.cl:227-248): rotate-half pairs (d, d + hd/2) with the host
// table row for the position ([hd/2] of {cos, sin}); no contraction, so it
// matches the oracle.
__device__ __forceinline__ float rope_cs(const float* m, int d, int half, float c, float s)
{
    if (d < half) return __fsub_rn(__fmul_rn(m[d], c), __fmul_rn(m[d + half], s));
    return __fadd_rn(__fmul_rn(m[d], c), __fmul_rn(m[d - half], s));
}

__device__ __forceinline__ float rope_one(const float* m, const float* row, int d, int half)
{
    const int fi = d < half ? d : d - half;
    return rope_cs(m, d, half, row[2 * fi], row[2 * fi + 1]);
}

int rmsnorm(Ctx* c, float* h, const float* delta, const uint16_t* gain, int n, float eps, float* out);
int add(Ctx* c, const float* a, const float* b, int n, float* out);
int silu_mul(Ctx* c, const float* g, const float* u, int n, float* out);
int rope_kv(Ctx* c, const float* q, const float* k, const float* v, const float* table, const int* pos,
            int n_heads, int n_kv, int hd, int max_ctx, float* q_out, uint16_t* kc, uint16_t* vc);
// one launch of the split-context attention (see k_attn)
// Workgroups per head (each a run of consecutive 64-position chunks; at most
// 32) up to which the model's attention adds its sums with fp64 atomics
// rather than through partial slots and a last workgroup: up to 32
// same-address adds per output cost less than the exchange, the arrival and
// the serial sum (measured per launch at 9 and 32 chains: 7.1 against 8.3 us
// and 12.9 against 13.5 us; at 61, 19.9 against 19.0 us).
constexpr int kAttnAtomicSplits = 40;

struct AttnLaunch {
    const float* q = nullptr;          // queries after RoPE, or null: from qkv_acc (RoPE and KV append applied)
    const void* qkv_acc = nullptr;
    int kv_copies = 1;                 // qkv_acc: 2 when k and v have second copies after v
    const float* rope = nullptr;
    uint16_t* kc = nullptr;
    uint16_t* vc = nullptr;
    const int* pos = nullptr;
    int n_heads = 0, n_kv = 0, max_ctx = 0;
    void* acc = nullptr;               // model: o then l (n_heads * 128 + n_heads doubles)
    // model: with at most this many workgroups per head, every one adds its
    // o and l into acc (which must be zero on entry) with fp64 atomics; with
    // more, the last workgroup of each head writes the sums
    int atomic_splits = 0;
    void* part = nullptr;              // the splits' partial sums (attention_part_words doubles)
    float* out = nullptr;              // standalone: out = o / l
    uint32_t* head_ctr = nullptr;      // [n_heads], zero on entry (left zero)
    void* zero_p = nullptr;
    int zero_n = 0;
};
int attention_launch(Ctx* c, const AttnLaunch& L);
size_t attention_acc_words(int n_heads);
// doubles of the per-split partials of one attention launch
size_t attention_part_words(int n_heads, int n_kv, int max_ctx);
// h_out = h + (float)delta accumulator (add32), then RMSNorm + gain into out
// (n = 1024 .. 16384, multiple of 1024); delta may be null
int resnorm(Ctx* c, const float* h, const void* delta_acc, float* h_out, const uint16_t* gain, int n, float eps,
            float* out);
int embed(Ctx* c, const uint16_t* table, int cols, int vocab, const int* tok, float* out);
// first-max argmax into out[0]; if pos_inc is non-null, *pos_inc += 1 and,
// when hist is non-null and the new position lies below hist_len,
// hist[new position] = the index
int argmax(Ctx* c, const float* v, int n, int* out, int* pos_inc, int* hist = nullptr, int hist_len = 0);
// matmul16x32 (aux.cl:454-490): out[r] = fp16 row r of W [rows][cols] times x,
// in the reference's work-group order (cols <= 16384)
int matmul_f16_dense(Ctx* c, const uint16_t* W, const float* x, int rows, int cols, float* out);

// synthetic data and the GPU bucketizer
int gen_f16(Ctx* c, uint64_t seed, uint64_t tid, size_t count, double mean, double sigma, uint16_t* out);
int gen_f32(Ctx* c, uint64_t seed, uint64_t tid, size_t count, double mean, double sigma, float* out);
int bucketize(Ctx* c, const uint16_t* w, int out_dim, int in_dim, uint16_t* buckets, uint16_t* stats,
              uint16_t* probes);

}  // namespace iam
