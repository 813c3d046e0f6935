/*
 * tinygiant.h -- C ABI of libtinygiant.so, the MI355X (gfx950) build of
 * TinyGiant's MoE expert hot path.
 *
 * Two groups of entry points:
 *
 *  1. The reference's own ABI (csrc/libtinygiant.c, registered by
 *     tinygiant/_lib.py:39-74), same names and C signatures, so that
 *     load_tinygiant_lib() binds this library unchanged.  Pointers are
 *     caller-owned host pointers and calls are synchronous, as in the
 *     reference.  Every one of them runs on the GPU (operands copied in per
 *     call, the new KV-cache rows copied back) with the reference's
 *     arithmetic order, bit-identical to its scalar definition with
 *     contraction off.  A failing call (these signatures return nothing)
 *     sets tg_last_error(), prints one line on stderr per symbol and writes
 *     NaN to every output element.
 *
 *  2. New entry points for the Q4_0/Q8_0 path: an all-experts-resident HBM
 *     arena (the reference's SSD/page-cache/mlock tiers collapsed into
 *     device memory with the same per-expert offsets) and whole-layer /
 *     whole-stack calls.  They return 0 on success and a negative TG_E*
 *     code on error; tg_last_error() describes the last error of the
 *     calling thread.  *_dev variants take device pointers and a HIP stream
 *     (hipStream_t passed as void*, NULL = null stream) and are
 *     asynchronous; the others take host pointers and synchronise.
 *
 * Formats: Q4_0 = {half d; u8 qs[16]} per 32 weights (element j < 16 is the
 * low nibble of qs[j], element j+16 the high nibble, value d*(q-8)); Q8_0 =
 * {half d; i8 qs[32]}.  An expert is gate[I x H] | up[I x H] | down[H x I]
 * and a layer is experts 0..E-1 back to back, exactly the bytes
 * tinygiant/relayout.py:142-157 writes; expert e starts at e * expert_bytes.
 */
#ifndef TINYGIANT_H
#define TINYGIANT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ */
/* error channel (new; the reference ABI has none)                      */
/* ------------------------------------------------------------------ */
#define TG_OK 0
#define TG_E_INVALID -1     /* bad argument: NULL, shape, range */
#define TG_E_NODEVICE -2    /* no HIP device / init failed */
#define TG_E_NOMEM -3       /* device allocation failed */
#define TG_E_HIP -4         /* a HIP runtime call failed */
#define TG_E_UNSUPPORTED -5 /* entry point not available in this build */

/* Message of the calling thread's last error ("" if none). */
const char *tg_last_error(void);
/* Select and initialise a HIP device (idempotent per device). */
int tg_gpu_init(int device);
/* Wait for all work on the device. */
int tg_device_sync(void);
/* Library version string. */
const char *tg_version(void);
/* Kernel timing.  While enabled, the MoE entry points bracket every kernel
 * launch with HIP events recorded on the launching stream; tg_prof_read
 * waits for them and returns, for one launch role ("dec_part", "layer",
 * "route", "route_q8", "group", "gu_down_mfma", "gateup_mfma", "down_mfma",
 * "combine", ...), the number of launches and their summed duration in ms.
 * tg_prof_enable(1) also discards earlier records. */
int tg_prof_enable(int on);
int tg_prof_read(const char *kernel, int *launches, double *total_ms);

/* ------------------------------------------------------------------ */
/* reference ABI (tinygiant/_lib.py:39-74)                              */
/* ------------------------------------------------------------------ */
/* csrc/libtinygiant.c:555 */
void tg_expert_forward(const uint8_t *q4_data, const float *input,
                       float *output, float weight,
                       int embed_dim, int inter_dim);
/* csrc/libtinygiant.c:599 */
void tg_expert_forward_mixed(const uint8_t *gate_q4, const uint8_t *up_q4,
                             const void *down_data, int down_format,
                             const float *input, float *output, float weight,
                             int embed_dim, int inter_dim);
/* csrc/libtinygiant.c:187 */
void tg_matmul_q4k(const uint8_t *q4_matrix, const float *input,
                   float *output, int nrows, int ncols);
/* csrc/libtinygiant.c:270 */
void tg_matmul_q6k(const uint8_t *q6_matrix, const float *input,
                   float *output, int nrows, int ncols);
/* csrc/libtinygiant.c:322 */
void tg_rms_norm(const float *x, const float *weight, float *out,
                 int dim, float eps);
/* csrc/libtinygiant.c:304 */
void tg_f32_matvec(const float *A, const float *x, float *out,
                   int nrows, int ncols);
/* csrc/libtinygiant.c:297 */
void tg_f16_matvec(const uint16_t *A, const float *x, float *out,
                   int nrows, int ncols);
/* csrc/libtinygiant.c:365 */
void tg_attention_decode(
    const float *wq, const float *wk, const float *wv, const float *wo,
    const float *q_norm_w, const float *k_norm_w,
    float *kv_k, float *kv_v, int kv_len, int kv_max,
    const float *rope_cos, const float *rope_sin,
    const float *input, float *output,
    int embed_dim, int n_heads, int n_kv_heads, int head_dim, int pos);
/* csrc/libtinygiant.c:460 */
void tg_attention_decode_q4(
    const uint8_t *wq_q4, const uint8_t *wk_q4,
    const uint16_t *wv_f16, const uint8_t *wo_q4,
    const float *q_norm_w, const float *k_norm_w,
    float *kv_k, float *kv_v, int kv_len, int kv_max,
    const float *rope_cos, const float *rope_sin,
    const float *input, float *output,
    int embed_dim, int n_heads, int n_kv_heads, int head_dim, int pos);
/* csrc/libtinygiant.c:745 */
void tg_prefetch(const void *addr, size_t len);
/* csrc/libtinygiant.c:752 */
void tg_prefetch_batch(const void **addrs, const size_t *lens, int count);
/* csrc/libtinygiant.c:761.  Returns mlock()'s result on the 16 KiB-aligned
 * range, as the reference.  The range may also be copied to HBM once
 * (tg_mirror_mode): by default when it lies wholly in mappings without write
 * permission, as the reference cache's mmap views of the relayout files
 * (cache.py:31-67); writable memory (the engine's attention weights,
 * engine.py:134-139) only in TG_MIRROR_ALL.  The legacy entry points then
 * read any weight operand lying inside a copied range from HBM instead of
 * copying it per call.  Each use first compares the range's first and last
 * 64 bytes and 16 words spread over it with what it held when locked (only
 * the parts inside the caller's operand are read); a mismatch drops the copy
 * and the call reads host memory. */
int tg_mlock(const void *addr, size_t len);
/* Release the HBM copies of every tg_mlock range overlapping
 * [addr, addr + len) (all of them for NULL), e.g. before unmapping or
 * rewriting it.  No counterpart in the reference (its locks live as long as
 * the process). */
void tg_mirror_drop(const void *addr, size_t len);
/* Bytes and ranges held in HBM for tg_mlock ranges, and how many legacy
 * weight operands were read from them (hits) or copied (misses).  Any
 * pointer may be NULL.  No counterpart in the reference. */
void tg_mirror_stats(size_t *bytes, int *ranges, uint64_t *hits, uint64_t *misses);
/* Which tg_mlock ranges are copied to HBM from now on: TG_MIRROR_OFF (none:
 * every legacy call reads host memory, as the reference), TG_MIRROR_READONLY
 * (the default: ranges wholly in read-only mappings), TG_MIRROR_ALL (also
 * writable memory; the caller promises that a locked range keeps its bytes
 * until tg_mirror_drop).  The environment variable TG_MLOCK_MIRROR (0, all)
 * sets the initial mode.  A negative mode only queries.  Returns the mode in
 * force, or TG_E_INVALID.  Copies already made are kept.  No counterpart in
 * the reference. */
#define TG_MIRROR_OFF 0
#define TG_MIRROR_READONLY 1
#define TG_MIRROR_ALL 2
int tg_mirror_mode(int mode);
/* csrc/libtinygiant.c:662 */
void tg_transformer_layer(
    const float *wq, const float *wk, const float *wv, const float *wo,
    const float *attn_norm_w, const float *q_norm_w, const float *k_norm_w,
    const float *ffn_norm_w,
    float *kv_k, float *kv_v, int kv_len, int kv_max,
    const float *rope_cos, const float *rope_sin,
    const uint8_t **gate_ptrs, const uint8_t **up_ptrs,
    const void **down_ptrs, const int *down_is_f16,
    const float *expert_weights, int n_active,
    float *x,
    int embed_dim, int inter_dim,
    int n_heads, int n_kv_heads, int head_dim, int pos);
/* csrc/libtinygiant.c:647 (exported, not registered by _lib.py) */
void tg_moe_forward(const uint8_t **expert_ptrs, const float *weights,
                    int n_experts, const float *input, float *output,
                    int embed_dim, int inter_dim);
/* csrc/libtinygiant.c:735 (exported, not registered by _lib.py) */
void tg_matmul_q4k_scalar(const uint8_t *q4_matrix, const float *input,
                          float *output, int nrows, int ncols);

/* ------------------------------------------------------------------ */
/* HBM expert arena (replaces tinygiant/cache.py's mmap/mlock tiers)    */
/* ------------------------------------------------------------------ */
typedef struct tg_arena tg_arena;

/* Reserve device memory for n_layers layers of n_experts Q4_0 experts plus
 * one fp32 router [n_experts x H] and one fp32 FFN norm weight [H] (all ones
 * until tg_arena_load_norm) per layer.  embed_dim = H must be a multiple of
 * 256 and inter_dim = I a multiple of 32, both at most 8192; n_experts a
 * multiple of 4 up to 252; top_k in 1..min(32, n_experts); the kernels'
 * LDS limits can refuse a shape within these bounds, and the error message
 * then says so.  Returns NULL on error (see tg_last_error).
 * Role: tinygiant/cache.py:14-57 (ExpertCache over index.json). */
tg_arena *tg_arena_create(int n_layers, int n_experts, int embed_dim,
                          int inter_dim, int top_k);
void tg_arena_destroy(tg_arena *a);
/* Bytes of one expert / one layer in the relayout format. */
size_t tg_arena_expert_bytes(const tg_arena *a);
size_t tg_arena_layer_bytes(const tg_arena *a);
/* Offset and gate/up/down sizes of expert e inside a layer, as recorded in
 * index.json's expert_offsets (relayout.py:150-156). */
int tg_arena_expert_offset(const tg_arena *a, int expert, size_t *offset,
                           size_t *gate_bytes, size_t *up_bytes,
                           size_t *down_bytes);
/* Upload one layer file's bytes (relayout layout, host memory). */
int tg_arena_load_layer(tg_arena *a, int layer, const void *host_bytes,
                        size_t nbytes);
/* Upload one layer's fp32 router [n_experts x H] (host memory). */
int tg_arena_load_router(tg_arena *a, int layer, const float *host_router,
                         size_t count);
/* Upload one layer's FFN norm weight [H] (host memory): the MoE block of
 * that layer runs on rms_norm(x) * w, as engine.py:229-230 does with
 * ffn_norms[i] (tg_rms_norm, csrc/libtinygiant.c:322-340).  The router is
 * applied as s * ((router * w) . x), the norm weight folded into the
 * router's columns once, here and in tg_arena_load_router. */
int tg_arena_load_norm(tg_arena *a, int layer, const float *host_norm,
                       size_t count);
/* Read one layer back in the relayout layout (host memory). */
int tg_arena_read_layer(tg_arena *a, int layer, void *host_bytes,
                        size_t nbytes);
/* Read one expert of one layer back (gate | up | down, relayout layout,
 * tg_arena_expert_bytes bytes).  Role: tinygiant/cache.py:154-160
 * (ExpertCache.get: one expert's views). */
int tg_arena_read_expert(tg_arena *a, int layer, int expert, void *host_bytes,
                         size_t nbytes);
/* Fill one layer (experts and router) with the synthetic workload on the
 * device: weights N(0, sigma) quantized to Q4_0, router N(0, sigma) fp32,
 * from SplitMix64 counters keyed by (seed, layer, expert, tensor). */
int tg_arena_synth_layer(tg_arena *a, int layer, uint64_t seed, float sigma);

/* ------------------------------------------------------------------ */
/* MoE block: norm -> router -> top-k -> experts -> combine             */
/* (engine.py:229-258 with Q4_0 experts)                                */
/* ------------------------------------------------------------------ */
/* For each of n_tokens tokens x[t] (fp32, H): xn = (x / rms(x)) * g (eps;
 * g the layer's norm weight), logits = router xn, top-k with renormalised
 * softmax, moe_out[t] = sum_j w_j * expert_j(Q8_0(xn)).  topk_idx / topk_w
 * ([n_tokens x k], descending logit) may be NULL. */
int tg_moe_layer_q40_dev(tg_arena *a, int layer, const float *x,
                         float *moe_out, int n_tokens, int32_t *topk_idx,
                         float *topk_w, float eps, void *stream);
/* The same on host buffers (x, moe_out, topk_idx, topk_w), synchronous.
 * Also returns TG_E_HIP when a device-side poll of its launch ran out of
 * tries (those rows are NaN), as tg_arena_status would. */
int tg_moe_layer_q40(tg_arena *a, int layer, const float *x, float *moe_out,
                     int n_tokens, int32_t *topk_idx, float *topk_w,
                     float eps);
/* tg_moe_layer_q40_dev that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, kernels and results as tg_moe_layer_q40_dev;
 * its scratch is a fixed 16 MiB device array per GPU, held until the
 * process ends, instead of the arena's.  Calls whose scratch would exceed it
 * fail with TG_E_INVALID (the message gives the largest n_tokens at the
 * arena's shape).  tg_gpu_init must have
 * run.  Every call on a GPU shares that GPU's array: calls that overlap on
 * one GPU (other streams, other threads) race.  Every call of one shape
 * uses the layout of the largest n_tokens that fits; each call first runs a
 * one-block kernel on `stream` that clears the array's exchange words when
 * the array last served another shape (the array's header records which, on
 * the device, so replays of a captured call decide the same way).  A poll
 * failure of these calls is reported by tg_arena_status on any arena. */
int tg_moe_layer_q40_noalloc_dev(tg_arena *a, int layer, const float *x,
                                 float *moe_out, int n_tokens,
                                 int32_t *topk_idx, float *topk_w, float eps,
                                 void *stream);
/* x <- x + MoE_l(x) for l = layer0 .. layer0+n_layers-1, in place.  The
 * decode path of one-token calls is chosen by tg_arena_set_decode_path. */
int tg_moe_stack_q40_dev(tg_arena *a, float *x, int n_tokens, int layer0,
                         int n_layers, float eps, void *stream);
/* (host buffer x, synchronous; returns what tg_arena_status then reports) */
int tg_moe_stack_q40(tg_arena *a, float *x, int n_tokens, int layer0,
                     int n_layers, float eps);
/* One token through layers layer0.. with the routing of every layer
 * recorded: topk_idx / topk_w are device arrays [n_layers x k]. */
int tg_moe_stack_q40_trace_dev(tg_arena *a, float *x, int layer0,
                               int n_layers, float eps, int32_t *topk_idx,
                               float *topk_w, void *stream);
/* Decode path of one-token calls: ROUTED (one launch per layer that also
 * routes, from router partial sums the layer before it leaves; stack
 * calls add one small prologue launch and launch layer by layer, or replay
 * as a HIP graph after tg_arena_set_graphs(a, 1)), FUSED
 * (per layer a routing kernel and one launch for gate/up and down),
 * PER_LAYER (routing, gate/up and down as three kernels per layer), AUTO
 * (ROUTED where the shape allows it, else FUSED, else PER_LAYER).  Value 1
 * is not a path (TG_E_INVALID).
 *
 * The ROUTED and FUSED launches hand data between their own blocks through
 * device memory (bounded polls), so they need every block of the launch
 * resident at once: H / rd blocks of 1024 threads, rd the smallest row
 * count that keeps the grid within the device's CUs (one block per CU).  Work that another stream
 * keeps on the same device can hold CUs for the whole launch; the polls then
 * run out of tries, the affected rows come back NaN and tg_arena_status()
 * reports the failure.  Run nothing else on the device beside these
 * launches. */
#define TG_DECODE_AUTO 0
#define TG_DECODE_PER_LAYER 2
#define TG_DECODE_FUSED 3
#define TG_DECODE_ROUTED 4
int tg_arena_set_decode_path(tg_arena *a, int path);
/* Path of calls over n_tokens > 1 tokens (batched decode, prefill):
 * GROUPED (the (token, slot) pairs grouped by expert, each selected
 * expert's weights read once per layer; int8 MFMA tiles), GROUPED_DOT (the
 * same grouping on packed int8 dot instructions), PER_TOKEN (every token
 * reads its own k experts), AUTO (GROUPED for n_tokens >= 2).  GROUPED and
 * GROUPED_DOT also serve a single token when asked for explicitly.  Every
 * path gives the same bytes. */
#define TG_BATCH_AUTO 0
#define TG_BATCH_GROUPED 1
#define TG_BATCH_PER_TOKEN 2
#define TG_BATCH_GROUPED_DOT 3
int tg_arena_set_batch_path(tg_arena *a, int path);
/* Stack calls (tg_moe_stack_q40*) launched layer by layer (on = 0, the
 * default; TG_GRAPH=1 in the environment makes 1 the default of new
 * arenas) or replayed as a HIP graph captured on the first call with the
 * same x, token count, layer range and eps (on = 1).  No counterpart in the
 * reference (it has no device graphs); on MI355X the direct launches of the
 * one-token and batched stacks measured 0.3-2.3% faster than the replay.
 * Both give the same bytes. */
int tg_arena_set_graphs(tg_arena *a, int on);
/* Waits for the device and reports a device-side failure of an earlier
 * asynchronous call on this arena, or of a no-alloc call on this device (a
 * hand-off poll of the ROUTED or FUSED launch, or a down block's wait in
 * the batched path's gate/up + down launch, that ran out of tries):
 * TG_E_HIP.  The failure is reported once: reading it clears it, and the
 * next calls run as before. */
int tg_arena_status(tg_arena *a);
/* Measurement, no counterpart in the reference: the shader clock (MHz)
 * while every CU runs int8 MFMA chains (four 256-thread blocks per CU,
 * `iters` rounds of four v_mfma_i32_16x16x32_i8 per wave), from each
 * block's shader-cycle and 100 MHz real-time counters: median, min, max
 * over the blocks (min / max may be NULL).  For the int8 peak at the clock
 * the MFMA kernels actually run at. */
int tg_clock_mfma_mhz(int iters, double *mhz_median, double *mhz_min,
                      double *mhz_max);
/* Test hook of the failure channel, no counterpart in the reference: the
 * poll bound of the ROUTED and FUSED launches and of the batched path's
 * gate/up + down launch (spin_limit tries; 0 restores the normal bound) and
 * one h line those launches leave unpublished (drop_line: a gate/up unit,
 * or half unit on shapes that split units, of the one-token launches; the
 * work item whose gate/up blocks never count in, in the batched launch; -1
 * none).  Every reader of that line then gives up after spin_limit tries,
 * each kernel exits normally, the rows come back NaN and the failure is
 * reported.  Not for production use. */
int tg_debug_fault_inject(uint32_t spin_limit, int drop_line);

/* ------------------------------------------------------------------ */
/* building blocks (device pointers; used by the parity tests)          */
/* ------------------------------------------------------------------ */
/* fp32 -> Q8_0 blocks (34 B each); n multiple of 32. */
int tg_q40_quantize_q8_0_dev(const float *x, void *q8_out, int n,
                             void *stream);
/* Relayout (18-byte block) tensor <-> the arena's tensor-planar form. */
int tg_q40_to_planar_dev(const void *aos, void *planar, int rows, int nb,
                         void *stream);
int tg_q40_from_planar_dev(const void *planar, void *aos, int rows, int nb,
                           void *stream);
/* Exact int32 block sums S[r][b] = sum (q_w - 8) q_x of a planar Q4_0
 * matrix [rows x cols] against Q8_0 blocks. */
int tg_q40_block_sums_dev(const void *w_planar, int rows, int cols,
                          const void *xq8, int32_t *sums, void *stream);
/* out[r] = Q4_0 row r . Q8_0 vector (planar matrix). */
int tg_q40_matvec_dev(const void *w_planar, int rows, int cols,
                      const void *xq8, float *out, void *stream);
/* Router logits (s * (Wr . x), grouped order) + top-k + softmax for
 * n_tokens; topk_idx / topk_w may be NULL.  Synchronous. */
int tg_router_topk_dev(const float *Wr, const float *x, int n_experts,
                       int embed_dim, int top_k, float eps, int n_tokens,
                       float *logits, int32_t *topk_idx, float *topk_w,
                       void *stream);
/* Measurement: one launch that reads nbytes (multiple of 16) of device
 * memory with plain 128-bit loads over `grid` 256-thread blocks; sink is one
 * device word.  The HBM read ceiling the expert kernels are compared with. */
int tg_stream_read_dev(const void *p, size_t nbytes, int grid, uint32_t *sink,
                       void *stream);
/* Synthetic generators (bit-identical to the host definition). */
int tg_synth_normal_dev(uint64_t seed, uint64_t stream_id, float sigma,
                        size_t n, float *out, void *stream);
int tg_synth_q40_dev(uint64_t seed, uint64_t stream_id, float sigma,
                     int rows, int cols, void *planar_out, void *stream);

/* Output head, the step after the layers (tinygiant/engine.py:262-266 forms
 * logits = output_weight @ rms_norm(x, output_norm) in numpy, and :359 takes
 * the greedy token np.argmax(logits)).  W [vocab][embed] fp32 and the norm
 * weight are copied to HBM once; each forward copies x in, runs the norm
 * (tg_rms_norm's order), the fp32 matvec (tg_f32_matvec's order,
 * libtinygiant.c:299-318) and the argmax (first index of the largest value,
 * NaN largest), and returns the token and, when logits is not NULL, the
 * vocab logits.  Create returns NULL on failure (tg_last_error() says why);
 * forward returns 0 or a negative TG_E_* code. */
typedef struct tg_head tg_head;
tg_head *tg_head_create(const float *W, const float *norm_w, int vocab, int embed);
int tg_head_forward(tg_head *h, const float *x, float eps, float *logits, int32_t *token);
void tg_head_destroy(tg_head *h);

/* Next-token sampling (tinygiant/engine.py:348-359, which samples in numpy
 * with np.random.choice).  temperature > 0: probs = exp((logits - max) / T)
 * normalised, the smallest prefix of the descending order (ties by
 * ascending id) whose float32 running sum reaches top_p (the crossing token
 * included; every token when it never does), those renormalised, and the
 * first one whose float64 cdf exceeds u.  u is the draw's uniform in [0, 1):
 * np.random.choice takes one RandomState.random_sample() per draw, so passing
 * that value reproduces the reference's token.  exp is the correctly rounded
 * fp32 value (numpy's float32 exp is within 2 ulp of it); every later step
 * follows numpy's operations and summation orders.  temperature <= 0 or NaN:
 * the greedy argmax (engine.py:359), and top_p, u and probs are unused.
 * Vocabularies up to 524288 tokens.  logits are a device pointer when
 * logits_on_device, else host memory; probs (host, vocab floats, may be NULL)
 * receives the normalised probabilities.  Calls return 0 or a negative
 * TG_E_* code: NaN or +inf logits, or all -inf, are TG_E_INVALID like a u
 * outside [0, 1).  No counterpart function in the reference. */
typedef struct tg_sampler tg_sampler;
tg_sampler *tg_sampler_create(int vocab);
int tg_sampler_run(tg_sampler *s, const float *logits, int logits_on_device, float temperature, double top_p,
                   double u, int32_t *token, float *probs);
void tg_sampler_destroy(tg_sampler *s);
/* tg_head_forward's logits sampled on the device (no logits copy needed;
 * logits may still be NULL or receive them). */
int tg_head_sample(tg_head *h, const float *x, float eps, float temperature, double top_p, double u,
                   float *logits, int32_t *token);

#ifdef __cplusplus
}
#endif
#endif
