// tg_internal.h -- shapes and kernel launchers shared by the C ABI layer.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tg {

// Kernel launch.  When a profiling caller has set g_launch_ev, the launch
// records those events at the kernel's own start and end
// (hipExtLaunchKernelGGL, the timestamps of the dispatch itself, as a kernel
// trace reports them) and clears them; otherwise it is hipLaunchKernelGGL.
struct LaunchEvents {
    hipEvent_t start, stop;
};
extern thread_local LaunchEvents g_launch_ev;
#define TG_LAUNCH(K, grid, block, lds, st, ...)                                                             \
    do {                                                                                                    \
        if (::tg::g_launch_ev.start) {                                                                      \
            const ::tg::LaunchEvents ev_ = ::tg::g_launch_ev;                                               \
            ::tg::g_launch_ev = {nullptr, nullptr};                                                         \
            hipExtLaunchKernelGGL(K, grid, block, (std::uint32_t)(lds), st, ev_.start, ev_.stop, 0u, __VA_ARGS__); \
        } else {                                                                                            \
            hipLaunchKernelGGL(K, grid, block, lds, st, __VA_ARGS__);                                       \
        }                                                                                                   \
    } while (0)

// One layer's geometry: H = embed dim, I = expert intermediate dim, E
// experts, top-k.  Byte sizes are those of the relayout format (18 bytes
// per 32 weights), which the planar arena keeps.
// n / d for n * d < 2^32 by one multiply-high: m = ceil(2^32 / d).
struct FastDiv {
    uint32_t d;
    uint64_t m;
};

inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f;
    f.d = d;
    f.m = ((1ull << 32) + d - 1) / d;
    return f;
}

__host__ __device__ inline uint32_t fdiv(uint32_t n, FastDiv f) { return (uint32_t)(((uint64_t)n * f.m) >> 32); }

struct Shape {
    int H, I, E, k;
    int nbH, nbI;      // blocks per gate/up row, per down row
    FastDiv divH, divI;
    size_t GB;         // bytes of gate (= up)
    size_t DB;         // bytes of down
    size_t EB;         // bytes of one expert
    size_t LB;         // bytes of one layer's experts
};

inline Shape make_shape(int H, int I, int E, int k) {
    Shape s;
    s.H = H; s.I = I; s.E = E; s.k = k;
    s.nbH = H / 32; s.nbI = I / 32;
    s.divH = make_fastdiv((uint32_t)s.nbH);
    s.divI = make_fastdiv((uint32_t)s.nbI);
    s.GB = (size_t)I * s.nbH * 18;
    s.DB = (size_t)H * s.nbI * 18;
    s.EB = 2 * s.GB + s.DB;
    s.LB = s.EB * (size_t)E;
    return s;
}

// Counter stream of one synthetic tensor: kind 0 gate, 1 up, 2 down,
// 3 router, 4 activations.
__host__ __device__ inline uint64_t stream_id(int layer, int expert, int kind) {
    return ((uint64_t)(layer & 0xFFFF) << 40) | ((uint64_t)(expert & 0xFFFFFF) << 8) | (uint64_t)(kind & 0xFF);
}

uint64_t host_stream_key(uint64_t seed, uint64_t stream);

// limits of the decode kernels
constexpr int MAX_K = 32;        // top-k
constexpr int MAX_E = 256;       // experts per layer (one thread per expert)
constexpr int MAX_NB = 256;      // blocks per row (H, I <= 8192)

// router[e][i] = raw[e][i] * g[i] (the FFN norm weight folded into the
// router: s * (router . x) is then the router applied to (x * s) * g)
hipError_t launch_scale_router(const float *raw, const float *g, float *router, int E, int H, hipStream_t st);
// every one of the n floats at p set to v
hipError_t launch_fill(float *p, float v, size_t n, hipStream_t st);
// one block: if *keyp != key, the n words at p are set to zero, then *keyp = key
hipError_t launch_keyed_clear(uint64_t *keyp, uint64_t key, uint32_t *p, size_t n, hipStream_t st);
hipError_t launch_synth_layer(uint8_t *layer_pl, float *router, const Shape &s, int layer,
                              uint64_t seed, float sigma, hipStream_t st);
hipError_t launch_synth_q40(uint8_t *pl, uint64_t key, float sigma, int rows, int nb, hipStream_t st);
hipError_t launch_synth_normal(float *out, uint64_t key, float sigma, size_t n, hipStream_t st);
hipError_t launch_repack_layer(const uint8_t *src, uint8_t *dst, const Shape &s, bool to_planar,
                               hipStream_t st);
hipError_t launch_repack_tensor(const uint8_t *src, uint8_t *dst, size_t nblocks, bool to_planar,
                                hipStream_t st);
hipError_t launch_quantize_q8_0(const float *x, uint8_t *out, int n, hipStream_t st);
hipError_t launch_block_sums(const uint8_t *w_pl, int rows, int nb, const uint8_t *xq8, int32_t *sums,
                             hipStream_t st);
hipError_t launch_matvec(const uint8_t *w_pl, int rows, int nb, const uint8_t *xq8, float *out,
                         hipStream_t st);
// routing: raw router dots (grouped order), then norm scale, logits, top-k
hipError_t launch_route(const float *Wr, const float *x, int T, int E, int H, float *raw, hipStream_t st);
hipError_t launch_topk(const float *raw, const float *x, int T, int E, int H, int k, float eps, float *logits,
                       int32_t *idx, float *w, hipStream_t st);
// decode MoE layer pieces
bool decode_shape_ok(const Shape &s);
// routing of T tokens in one launch: lw [T][E] tagged logits, ctl [T][2]
// (word 1: generation of the token's last routing; zero before first use),
// err set to nonzero when a poll ran out of tries; writes idx, w [T][k]
// and the Q8_0 activations xq [T][H], xd / xs [T][H/32]
// (gn: the FFN norm weight, H floats; the expert input is Q8_0((x * s) * gn))
hipError_t launch_route_dec(const float *Wr, const float *x, const float *gn, int T, const Shape &s, float eps,
                            uint64_t *lw, uint32_t *ctl, uint32_t *err, int32_t *idx, float *w, int8_t *xq, float *xd,
                            int *xs, hipStream_t st);
// gate/up + SwiGLU -> Q8_0 h [T][k][I] (hd / hs [T][k][I/32])
hipError_t launch_gateup(const uint8_t *layer_pl, const Shape &s, int T, const int32_t *idx, const int8_t *xq,
                         const float *xd, const int *xs, int8_t *hq, float *hd, int *hs, hipStream_t st);
// one token: gate/up and down in one launch (h handed over as hw tagged
// words, experts_fused_words of them, zero before first use; tags from the
// routing generation ctl[1])
bool experts_fused_ok(const Shape &s, int n_cu);
size_t experts_fused_words(const Shape &s);

// Legacy formats (libtinygiant.c): 256-value super-blocks; Q4_K 144 bytes,
// Q6_K 210 bytes, the Q8 activation block (fp32 scale, int32 sum, 256 int8)
// 264 bytes.  Launchers of tg_legacy.hip; xq buffers are 8-byte aligned,
// Q4_K matrices 16-byte aligned.
constexpr int LG_QK = 256, LG_Q4K_BYTES = 144, LG_Q6K_BYTES = 210, LG_Q8K_BYTES = 264;
hipError_t launch_quantize_q8k(const float *x, void *xq, int nblocks, hipStream_t st);
hipError_t launch_matmul_q4k(const uint8_t *W, const void *xq, float *y, int nrows, int bpr, hipStream_t st);
hipError_t launch_matmul_q6k(const uint8_t *W, const void *xq, float *y, int nrows, int bpr, hipStream_t st);
hipError_t launch_matvec_two_acc(const void *A, bool half, const float *x, float *y, int nrows, int ncols,
                                 hipStream_t st);
hipError_t launch_rms_norm(const float *x, const float *w, float *out, int dim, float eps, hipStream_t st);
hipError_t launch_matmul_q4k_scalar(const uint8_t *W, const float *x, float *y, int nrows, int bpr, hipStream_t st);
hipError_t launch_silu_mul_vec(const float *g, const float *u, float *h, int n, hipStream_t st);
hipError_t launch_acc_scaled(float *out, const float *v, float w, int n, hipStream_t st);
// tg_moe_forward's experts in three launches (after the Q8 of x): device
// pointers of each expert's gate, up and down (Q4_K) and its weight
constexpr int LG_MOE_MAX = 16;
struct LgMoeOps {
    const uint8_t *gate[LG_MOE_MAX], *up[LG_MOE_MAX], *down[LG_MOE_MAX];
    float w[LG_MOE_MAX];
};
// gu: n_exp * 2 * inter floats (every expert's gate then up rows), hq:
// n_exp * inter / 256 Q8 blocks of SiLU(gate) * up; out: embed floats,
// written (not added to)
// shapes the fused launches take: 1 .. LG_MOE_MAX experts, embed and inter
// multiples of 256, embed at most 32768
bool moe_q4k_ok(int n_exp, int embed, int inter);
// (x: the fp32 input; each block forms its Q8 blocks in LDS)
hipError_t launch_moe_gateup_q4k(const LgMoeOps &P, int n_exp, const float *x, float *gu, int embed, int inter,
                                 hipStream_t st);
hipError_t launch_moe_silu_q8k(const float *gu, void *hq, int n_exp, int inter, hipStream_t st);
hipError_t launch_moe_down_acc_q4k(const LgMoeOps &P, int n_exp, const void *hq, float *out, int embed, int inter,
                                   bool add_to_out,
                                   hipStream_t st);
hipError_t launch_rms_norm_rows(const float *x, const float *w, float *out, int dim, int rows, float eps,
                                hipStream_t st);
hipError_t launch_rope(float *x, int n_heads, int hd, const float *c, const float *sn, hipStream_t st);
hipError_t launch_kv_append(const float *kn, const float *v, float *kc, float *vc, int n_kv, int seq, int hd, int row,
                            hipStream_t st);
// Attention of n_heads query heads over seq cached positions, caches
// [n_kv][seq][hd] (ratio = n_heads / n_kv query heads per kv head), hd <= 512,
// in three launches: scores and per-block maxima, the softmax weights of each
// head, the weighted sum of V into out.  scr holds attn_scratch_floats()
// floats: [n_heads][seq] scores, [n_heads][nblk] maxima, then (from a 16-byte
// boundary) [n_heads][seq rounded up to 4] weights.
constexpr int ATT_HB = 8;   // query heads of one kv head per block
constexpr int ATT_TP = 16;  // positions per scores block
inline int attn_score_blocks(int seq) { return (seq + ATT_TP - 1) / ATT_TP; }
inline size_t attn_w_offset(int n_heads, int seq) {
    return ((size_t)n_heads * ((size_t)seq + attn_score_blocks(seq)) + 3) & ~(size_t)3;
}
inline size_t attn_scratch_floats(int n_heads, int seq) {
    return attn_w_offset(n_heads, seq) + (size_t)n_heads * (((size_t)seq + 3) & ~(size_t)3);
}
hipError_t launch_attn_scores(const float *q, const float *kc, float *scr, int n_heads, int seq, int hd, int ratio,
                              float inv_sqrt, hipStream_t st);
hipError_t launch_attn_softmax(float *scr, int n_heads, int seq, hipStream_t st);
hipError_t launch_attn_wv(const float *scr, const float *vc, float *out, int n_heads, int seq, int hd, int ratio,
                          hipStream_t st);
hipError_t launch_add_vec(float *x, const float *a, int n, hipStream_t st);
// first index of the largest of x[0..n) (NaN largest) into out[0]; pv / pi
// hold ARGMAX_BLOCKS partials
constexpr int ARGMAX_BLOCKS = 256;
hipError_t launch_argmax(const float *x, int n, float *pv, int *pi, int *out, hipStream_t st);

// Temperature / top-p sampling (tg_sample.hip).
constexpr int SMP_VMAX = 1 << 19;        // largest vocabulary
constexpr int SMP_BUCKETS = 4096;        // histogram over q's bits 30..19
constexpr int SMP_BUCKET_SHIFT = 19;
constexpr int SMP_SMALL = 8192;          // candidates sorted in one block's LDS
constexpr int NP_BUFSIZE = 8192;         // np.sum reduces in buffers of this many values
constexpr int SMP_ST_PENDING = -1, SMP_ST_OK = 0, SMP_ST_INPUT = 1, SMP_ST_BOUND = 2;
struct SmpCtl {
    float m, S;        // max logit, np.sum of p
    int bad;           // a NaN or +inf logit, or every logit -inf
    int bstar;         // lowest histogram bucket of the candidate prefix
    uint32_t C;        // elements in buckets >= bstar
    uint32_t n;        // compaction counter
    uint32_t done;     // blocks of the histogram launch that have finished
    int large;         // C > SMP_SMALL: the sort runs in global memory
    int cut;           // candidates after the top-p cutoff
    int token;
    int status;        // SMP_ST_*
};
struct SmpBufs {
    float *pmax;                  // 256 block maxima
    int *pbad;                    // 256 block flags
    float *p, *q;                 // vocab: exp values, probabilities
    float *sums;                  // 64 buffer sums
    uint32_t *hcnt;               // SMP_BUCKETS
    unsigned long long *hmass;    // SMP_BUCKETS
    unsigned long long *keys;     // next power of two >= max(vocab, 16384)
    float *sq;                    // vocab: sorted probabilities (more than SMP_SMALL candidates)
    uint32_t *sid;                // vocab: their token ids
    SmpCtl *ctl;
};
hipError_t sample_prepare();
// k_smp_max .. k_smp_small; afterwards ctl->large says whether launch_sample_large must finish
hipError_t launch_sample_main(const SmpBufs &b, const float *logits, int V, float T, double top_p, double u,
                              hipStream_t st);
hipError_t launch_sample_large(const SmpBufs &b, int V, int C, double top_p, double u, hipStream_t st);

// One-token layer with routing inside (k_layer_dec) and the prologue that
// forms the first layer's router partials (k_dec_part).  part buffers hold
// [E+1][H/32] floats, dec_part_floats() the size of two; the group hand-off
// takes dec_ow_words() tagged words.
bool layer_dec_ok(const Shape &s, int n_cu);
size_t dec_part_floats(const Shape &s);
size_t dec_ow_words(const Shape &s);
hipError_t launch_dec_part(const float *Wr, const float *x, const Shape &s, float *part, uint32_t *ctl, int n_layers,
                           hipStream_t st);
hipError_t launch_layer_dec(const uint8_t *layer_pl, const Shape &s, int n_cu, const float *x, const float *gn,
                            const float *part_in, const float *wr_next, float *part_out, uint64_t *hw, uint64_t *ow,
                            const uint32_t *ctl, uint32_t back, uint32_t *err, const float *resid, float *out,
                            int32_t *idx, float *w, float eps, hipStream_t st);
hipError_t launch_experts_fused(const uint8_t *layer_pl, const Shape &s, int n_cu, const int32_t *idx, const float *w,
                                const int8_t *xq, const float *xd, const int *xs, uint64_t *hw, const uint32_t *ctl,
                                uint32_t *err, const float *resid, float *out, hipStream_t st);
// down + combine (+ resid) -> out [T][H]
hipError_t launch_down(const uint8_t *layer_pl, const Shape &s, int T, const int32_t *idx, const float *w,
                       const int8_t *hq, const float *hd, const int *hs, const float *resid, float *out,
                       hipStream_t st);

// Failure-channel test hook: poll bound of the one-token expert launches
// (0: the normal bound) and one h line they leave unpublished (-1: none).
void set_fault_injection(uint32_t spin_limit, int drop_line);

// shader clock under int8 MFMA load: out[4 * block] = s_memtime, s_memrealtime
// (100 MHz) before, and both after, `iters` rounds of four MFMA chains
hipError_t launch_clock_mfma(unsigned long long *out, int blocks, int iters, hipStream_t st);

hipError_t launch_stream_read(const void *p, size_t bytes, int grid, uint32_t *sink, hipStream_t st);

// grouped (batched decode / prefill) MoE layer pieces
bool grouped_shape_ok(const Shape &s);
// raw [T][E] router dots, or chains [H/32][T][E] (non-null: summed first)
// ent_cap non-null: each token's k entries also go into per-expert lists
// ent_cap[e * T + i] (i from the atomic count ecnt[e], zero before the call)
// G.arrive non-null (with ent_cap): the last block to finish also builds the
// work items of the placed lists (items of at most G.ch entries, both lists
// alike, at most G.wmax each), clears ecnt and G.rdy (may be null) and sets
// *G.arrive (one word, zero between calls) back to zero: the grouping
// kernel's work in the same launch.
struct RouteGroup {
    int32_t *counts = nullptr, *offsets = nullptr, *work = nullptr, *work_n = nullptr, *rdy = nullptr;
    uint32_t *arrive = nullptr;
    int ch = 0, wmax = 0;
};
hipError_t launch_route_q8(const float *raw, const float *chains, const float *x, const float *gn, int T, int E,
                           int H, int k, float eps, int32_t *idx, float *w, int8_t *xq, float *xd, int *xs,
                           int32_t *ecnt, int32_t *ent_cap, const RouteGroup &G, hipStream_t st);
// TG_ROUTE_GROUP not 0 (read per call): route_q8 builds the placed lists'
// one-tile work items itself
bool route_groups_on();
// Few tokens: the router's per-group fma chains [H/32][T][E], for
// launch_route_q8 to add (T < 128, E <= 128 and a multiple of 32).
bool route_chains_usable(int T, int E, int H);
hipError_t launch_route_chains(const float *Wr, const float *x, int T, int E, int H, float *chains, hipStream_t st);
// work list: at most group_work_max(s, n) items per list, two lists
int group_work_max(const Shape &s, int n);
int group_work_max(const Shape &s, int n, int ch);
// rdy (may be null): one word per work item, zeroed for launch_gu_down_ms
hipError_t launch_group_chunked(const Shape &s, const int32_t *idx, int n, int ch, int32_t *counts,
                                int32_t *offsets, int32_t *entries, int32_t *work, int32_t *work_n, int32_t *rdy,
                                hipStream_t st);
// Many entries: idx[n] placed into per-expert lists ent_cap[e * cap + i] by
// many blocks (counts in ecnt, zero before the call); the last block builds
// the work items of both lists (chunks of G.ch entries, largest first),
// clears ecnt and G.rdy (may be null) and sets *G.arrive (zero between calls)
// back to zero.  TG_GROUP_PAR not 0 (read per call)
bool place_par_on();
hipError_t launch_place(const int32_t *idx, int n, int E, int cap, int32_t *ecnt, int32_t *ent_cap,
                        const RouteGroup &G, hipStream_t st);
// work items over entries placed by launch_route_q8 (lists of capacity cap);
// clears ecnt for the next call
hipError_t launch_group_placed(const Shape &s, int n, int ch, int cap, int32_t *ecnt, int32_t *counts,
                               int32_t *offsets, int32_t *work, int32_t *work_n, int32_t *rdy, hipStream_t st);
// int8-MFMA grouped gate/up and down (mt = M-tiles of 32 entries per item)
bool mfma_shape_ok(const Shape &s);
int mfma_tiles(const Shape &s, int T);
// entries per work item for the MFMA launches at mt M-tiles
int mfma_item_entries(const Shape &s, int mt);
hipError_t launch_gateup_mfma(const uint8_t *layer_pl, const Shape &s, int mt, int wmax, const int32_t *work,
                              const int32_t *work_n, const int32_t *entries, const int8_t *xq, const float *xd,
                              const int *xs, int8_t *hq, float *hd, int *hs, hipStream_t st);
// The combine folded into the down launch: w [T][k] routing weights, resid
// (may be null) and out [T][H], and cnt, one arrival count per (token, tile of
// FC_ROWS output rows), zero between calls (the down launch leaves them zero).
constexpr int FC_ROWS = 128;
struct FuseArgs {
    const float *w = nullptr;
    const float *resid = nullptr;
    float *out = nullptr;
    uint32_t *cnt = nullptr;  // null: no combine in the down launch
};
inline size_t fuse_count_words(const Shape &s, int T) { return (size_t)T * (size_t)(s.H / FC_ROWS); }
// The down launch at mt M-tiles combines too (FuseArgs honoured): its kernel
// takes whole FC_ROWS-row tiles (H % FC_ROWS == 0) and TG_FUSE_COMBINE is 1.
bool down_fuses(const Shape &s, int mt, int T);
// Gate/up and down of one-tile work items in one launch (k_mfma_small_gd):
// rdy holds one word per work item, zero at the launch (the grouping kernel
// clears them); a down block whose wait for its item's h runs out of tries
// stores NaN rows and sets *err to 4.
struct GdArgs {
    int32_t *rdy = nullptr;
    uint32_t *err = nullptr;
    uint32_t spin = 0;  // poll bound
    int drop = -1;      // failure-channel hook: the item whose gate/up blocks never count in
    int need = 0;       // gate/up blocks per item (set by the launcher)
};
// the fused launch applies: one-tile items (mt == 1), the down K at most 8
// chunks of 8 blocks, and TG_FUSE_GD not 0 (read per call)
bool gd_fuses(const Shape &s, int mt);
hipError_t launch_gu_down_ms(const uint8_t *layer_pl, const Shape &s, int wmax, const int32_t *work,
                             const int32_t *work_n, const int32_t *entries, const int8_t *xq, const float *xd,
                             int8_t *hq, float *hd, int *hs, float *D, const GdArgs &G, hipStream_t st);
// The same for the 16 x 16 items (mt == 4 with items of more than 128
// entries: prefill and large batches); TG_FUSE_GD16 not 0 (read per call)
bool gd16_fuses(const Shape &s, int mt);
hipError_t launch_gu_down_x16(const uint8_t *layer_pl, const Shape &s, int wmax, const int32_t *work,
                              const int32_t *work_n, const int32_t *entries, const int8_t *xq, const float *xd,
                              int8_t *hq, float *hd, int *hs, float *D, const GdArgs &G, hipStream_t st);
// the poll bound and the withheld line / item of the failure-channel hook
uint32_t poll_spin_limit();
int poll_drop();
hipError_t launch_down_mfma(const uint8_t *layer_pl, const Shape &s, int mt, int wmax, const int32_t *work,
                            const int32_t *work_n, const int32_t *entries, const int8_t *hq, const float *hd,
                            const int *hs, float *D, const FuseArgs &F, hipStream_t st);
hipError_t launch_group(const Shape &s, const int32_t *idx, int n, int32_t *counts, int32_t *offsets,
                        int32_t *entries, int32_t *work, int32_t *work_n, hipStream_t st);
hipError_t launch_gateup_grouped(const uint8_t *layer_pl, const Shape &s, int n, const int32_t *work,
                                 const int32_t *work_n, const int32_t *entries, const int8_t *xq, const float *xd,
                                 const int *xs, int8_t *hq, float *hd, int *hs, hipStream_t st);
hipError_t launch_down_grouped(const uint8_t *layer_pl, const Shape &s, int n, const int32_t *work,
                               const int32_t *work_n, const int32_t *entries, const int8_t *hq, const float *hd,
                               const int *hs, float *D, hipStream_t st);
hipError_t launch_combine(const float *D, const float *w, int T, int H, int k, const float *resid, float *out,
                          hipStream_t st);

}  // namespace tg
