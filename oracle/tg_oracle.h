/*
 * tg_oracle.h -- CPU restatement of TinyGiant's MoE expert hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: pytest (tests/),
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product library (tinygiant_amd/libtinygiant.so) never links or calls it.
 *
 * Formats (all little-endian):
 *   Q4_0 block  = { u16 d (IEEE half); u8 qs[16] }        18 B / 32 weights
 *                 element j<16 = qs[j] & 15, element j+16 = qs[j] >> 4,
 *                 value = d * (q - 8)
 *   Q8_0 block  = { u16 d (IEEE half); i8 qs[32] }        34 B / 32 values
 *   Expert      = gate[I x H] | up[I x H] | down[H x I], each row-major in
 *                 Q4_0 blocks along the row; the layer file is experts
 *                 0..E-1 back to back (tinygiant/relayout.py:142-157).
 *
 * Every floating-point step is written out (explicit fmaf, no contraction:
 * compile with -ffp-contract=off) so that the GPU kernels, which perform the
 * same steps in the same order, produce bit-identical results.
 *
 * Parity status of each function is stated at its definition in
 * tg_oracle.c together with the test that pins it.
 */
#ifndef TG_ORACLE_H
#define TG_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TGO_QK 32
#define TGO_Q40_BYTES 18
#define TGO_Q80_BYTES 34

/* ---- scalar conversions and math ---- */
float    tgo_f16_to_f32(uint16_t h);
void     tgo_f16_to_f32_n(const uint16_t *h, size_t n, float *out);
uint16_t tgo_f32_to_f16(float f);
float    tgo_expf(float x);
float    tgo_ln_unit(float u);
float    tgo_cos2pi(float u);

/* ---- synthetic data (counter-based, thread-count independent) ---- */
uint64_t tgo_splitmix64(uint64_t x);
uint64_t tgo_stream_key(uint64_t seed, uint64_t stream);
float    tgo_normal_at(uint64_t key, uint64_t index);
void     tgo_synth_normal(uint64_t seed, uint64_t stream, float sigma,
                          size_t n, float *out);
void     tgo_synth_q40(uint64_t seed, uint64_t stream, float sigma,
                       int rows, int cols, uint8_t *out);

/* ---- Q4_0 / Q8_0 ---- */
void    tgo_quantize_q4_0(const float *x, size_t n, uint8_t *out);
void    tgo_dequantize_q4_0(const uint8_t *q, size_t n, float *out);
void    tgo_quantize_q8_0(const float *x, size_t n, uint8_t *out);
void    tgo_dequantize_q8_0(const uint8_t *q, size_t n, float *out);
int32_t tgo_block_dot_q40_q80(const uint8_t *w, const uint8_t *x);
void    tgo_block_sums(const uint8_t *W, int rows, int cols,
                       const uint8_t *xq, int32_t *sums);
float   tgo_row_dot_q40_q80(const uint8_t *wrow, const uint8_t *xq, int nb);
void    tgo_matvec_q40(const uint8_t *W, int rows, int cols,
                       const uint8_t *xq, float *out);
void    tgo_q40_to_planar(const uint8_t *aos, int rows, int nb, uint8_t *pl);
void    tgo_q40_from_planar(const uint8_t *pl, int rows, int nb, uint8_t *aos);

/* ---- norm, router, SwiGLU, expert, layer, stack ---- */
float   tgo_sumsq(const float *x, int n);
float   tgo_rms_scale(const float *x, int n, float eps);
float   tgo_router_dot(const float *w, const float *xn, int n);
void    tgo_router_logits(const float *Wr, int E, int H, const float *x,
                          float s, float *logits);
void    tgo_topk_softmax(const float *logits, int E, int k,
                         int32_t *idx, float *w);
float   tgo_silu_mul(float g, float u);
void    tgo_expert_q40(const uint8_t *expert, int H, int I,
                       const uint8_t *xq, float *gate, float *up,
                       float *h, uint8_t *hq, float *down);
float   tgo_router_dot_g(const float *w, const float *g, const float *x, int n);
void    tgo_moe_layer_q40(const uint8_t *layer, const float *Wr,
                          const float *g, int H, int I, int E, int k,
                          float eps, const float *x, int n_tokens,
                          float *moe_out, int32_t *idx, float *w,
                          uint8_t *xq_out);
void    tgo_moe_stack_q40(const uint8_t *const *layers,
                          const float *const *routers,
                          const float *const *norms, int n_layers,
                          int H, int I, int E, int k, float eps,
                          float *x, int n_tokens, int32_t *idx_trace);
int     tgo_group_by_expert(const int32_t *idx, int n_tokens, int k, int E,
                            int32_t *counts, int32_t *offsets,
                            int32_t *perm);

/* ---- legacy Q4_K / Q6_K / f16 functions (libtinygiant.c ABI) ---- */
typedef struct { float scale; int32_t sum; int8_t qs[256]; } tgo_q8k_block;
void  tgo_quantize_q8k(const float *x, tgo_q8k_block *out, int n_blocks);
void  tgo_scale_min_k4(int j, const uint8_t *scales, uint8_t *sc, uint8_t *m);
float tgo_dot_q4k_q8(const uint8_t *q4, const tgo_q8k_block *xq, int bpr);
void  tgo_matmul_q4k(const uint8_t *W, const float *x, float *y,
                     int nrows, int ncols);
float tgo_dot_q6k_q8(const uint8_t *q6, const tgo_q8k_block *xq, int bpr);
void  tgo_matmul_q6k(const uint8_t *W, const float *x, float *y,
                     int nrows, int ncols);
void  tgo_matvec_f16(const uint16_t *A, const float *x, float *y,
                     int nrows, int ncols);
void  tgo_matvec_f32(const float *A, const float *x, float *y,
                     int nrows, int ncols);
void  tgo_rms_norm(const float *x, const float *w, float *out, int dim,
                   float eps);
void  tgo_expert_forward_mixed(const uint8_t *gate, const uint8_t *up,
                               const void *down, int down_format,
                               const float *in, float *out, float weight,
                               int embed, int inter);
void  tgo_moe_forward_q4k(const uint8_t *const *experts, const float *w,
                          int n, const float *in, float *out,
                          int embed, int inter);
void  tgo_matmul_q4k_scalar(const uint8_t *W, const float *x, float *y,
                            int nrows, int ncols);
void  tgo_dequant_q4k_block(const uint8_t *block, float *out);
void  tgo_dequant_q6k_block(const uint8_t *block, float *out);

void  tgo_rope(float *x, int n_heads, int head_dim, const float *cos_t, const float *sin_t, int pos);
void  tgo_attention_decode(const float *wq, const float *wk, const float *wv, const float *wo,
                           const float *q_norm_w, const float *k_norm_w, float *kv_k, float *kv_v,
                           int kv_len, int kv_max, const float *rope_cos, const float *rope_sin,
                           const float *input, float *output, int embed, int n_heads,
                           int n_kv_heads, int head_dim, int pos);
void  tgo_attention_decode_q4(const uint8_t *wq, const uint8_t *wk, const uint16_t *wv,
                              const uint8_t *wo, const float *q_norm_w, const float *k_norm_w,
                              float *kv_k, float *kv_v, int kv_len, int kv_max,
                              const float *rope_cos, const float *rope_sin, const float *input,
                              float *output, int embed, int n_heads, int n_kv_heads,
                              int head_dim, int pos);
void  tgo_transformer_layer(const float *wq, const float *wk, const float *wv, const float *wo,
                            const float *attn_norm_w, const float *q_norm_w,
                            const float *k_norm_w, const float *ffn_norm_w, float *kv_k,
                            float *kv_v, int kv_len, int kv_max, const float *rope_cos,
                            const float *rope_sin, const uint8_t *const *gate_ptrs,
                            const uint8_t *const *up_ptrs, const void *const *down_ptrs,
                            const int *down_is_f16, const float *expert_weights, int n_active,
                            float *x, int embed, int inter, int n_heads, int n_kv_heads,
                            int head_dim, int pos);

/* ---- threading for the CPU baseline (no effect on results) ---- */
int   tgo_set_threads(int n);
int   tgo_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
