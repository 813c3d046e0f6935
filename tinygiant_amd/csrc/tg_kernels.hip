// tg_kernels.hip -- gfx950 kernels of the Q4_0 MoE expert path.
//
// Arena layout.  A layer holds experts 0..E-1 at e * expert_bytes, each
// expert gate | up | down at the byte offsets of the relayout file
// (tinygiant/relayout.py:142-157).  Inside each tensor the bytes are
// tensor-planar: the 16 nibble bytes of every block in (row, block) order,
// then the half scales in the same order.  A nibble group is then one
// aligned 128-bit load and a run of consecutive (row, block) pairs is
// contiguous, which the 18-byte relayout blocks are not.
//
// Per-row arithmetic (every path computes it identically):
//   S_b  = sum_i (q_w - 8) q_x                  exact int32
//   acc  = fma(round(S_b * dw_b), dx_b, acc)    b = 0 .. nb-1, acc0 = 0
// A tile first forms round(S_b * dw_b) for all its (row, block) pairs in
// parallel into LDS, then one lane per row runs the sequential fma chain.
#include "tg_device.h"
#include "tg_internal.h"

#include <limits.h>

namespace tg {

// ================================================================== shapes
struct TensorRef {
    int tensor;    // 0 gate, 1 up, 2 down
    int rows, nb;  // rows and blocks per row
    size_t off;    // byte offset of the tensor inside the expert
    size_t local;  // block index inside the tensor
};

TG_DEV TensorRef locate_block(const Shape &s, size_t rem) {
    TensorRef t;
    size_t gblocks = (size_t)s.I * s.nbH;
    if (rem < gblocks) {
        t.tensor = 0; t.rows = s.I; t.nb = s.nbH; t.off = 0; t.local = rem;
    } else if (rem < 2 * gblocks) {
        t.tensor = 1; t.rows = s.I; t.nb = s.nbH; t.off = s.GB; t.local = rem - gblocks;
    } else {
        t.tensor = 2; t.rows = s.H; t.nb = s.nbI; t.off = 2 * s.GB; t.local = rem - 2 * gblocks;
    }
    return t;
}

// ====================================================== synthetic weights
// Q4_0 rule on 32 values (signed max m, d = m/-8, q = min(15, trunc(x/d +
// 8.5))), stored planar.
TG_DEV void quant_q40_store(const float *v, uint8_t *qs_dst, uint16_t *d_dst) {
    float amax = 0.0f, vmax = 0.0f;
#pragma unroll
    for (int j = 0; j < QK; j++) {
        float a = fabsf(v[j]);
        if (amax < a) { amax = a; vmax = v[j]; }
    }
    float d = vmax / -8.0f;
    float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    uint32_t wv[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t word = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            int j = 4 * k + c;
            int q0 = (int)(v[j] * id + 8.5f);
            int q1 = (int)(v[j + 16] * id + 8.5f);
            q0 = q0 > 15 ? 15 : q0;
            q1 = q1 > 15 ? 15 : q1;
            word |= (uint32_t)(q0 | (q1 << 4)) << (8 * c);
        }
        wv[k] = word;
    }
    *reinterpret_cast<uint4 *>(qs_dst) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
    *d_dst = f2h(d);
}

// One thread per Q4_0 block of the layer: 32 draws, quantize, store.
__global__ __launch_bounds__(256) void k_synth_layer(uint8_t *__restrict__ layer_pl, Shape s,
                                                     uint64_t seed, int layer, float sigma,
                                                     size_t nblocks) {
    size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= nblocks) return;
    size_t bpe = (size_t)2 * s.I * s.nbH + (size_t)s.H * s.nbI;
    int e = (int)(g / bpe);
    TensorRef t = locate_block(s, g - (size_t)e * bpe);
    uint64_t key = stream_key(seed, stream_id(layer, e, t.tensor));
    size_t r = t.local / (size_t)t.nb, b = t.local - r * (size_t)t.nb;
    uint64_t base = (uint64_t)r * (uint64_t)t.nb * QK + (uint64_t)b * QK;
    float v[QK];
#pragma unroll
    for (int j = 0; j < QK; j++) v[j] = sigma * normal_at(key, base + (uint64_t)j);
    uint8_t *tb = layer_pl + (size_t)e * s.EB + t.off;
    size_t nt = (size_t)t.rows * t.nb;
    quant_q40_store(v, tb + t.local * 16, reinterpret_cast<uint16_t *>(tb + nt * 16) + t.local);
}

__global__ __launch_bounds__(256) void k_synth_q40(uint8_t *__restrict__ pl, uint64_t key, float sigma,
                                                   int rows, int nb) {
    size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t n = (size_t)rows * nb;
    if (g >= n) return;
    size_t r = g / (size_t)nb, b = g - r * (size_t)nb;
    uint64_t base = (uint64_t)r * (uint64_t)nb * QK + (uint64_t)b * QK;
    float v[QK];
#pragma unroll
    for (int j = 0; j < QK; j++) v[j] = sigma * normal_at(key, base + (uint64_t)j);
    quant_q40_store(v, pl + g * 16, reinterpret_cast<uint16_t *>(pl + n * 16) + g);
}

__global__ __launch_bounds__(256) void k_synth_normal(float *__restrict__ out, uint64_t key, float sigma,
                                                      size_t n) {
    size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g < n) out[g] = sigma * normal_at(key, g);
}

// ================================================================= repack
// relayout 18-byte blocks <-> tensor-planar, one thread per block.
TG_DEV void aos_to_planar_block(const uint8_t *src, uint8_t *qs_dst, uint16_t *d_dst) {
    const uint16_t *s16 = reinterpret_cast<const uint16_t *>(src);  // blocks are 2-byte aligned
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; k++) w[k] = (uint32_t)s16[1 + 2 * k] | ((uint32_t)s16[2 + 2 * k] << 16);
    *reinterpret_cast<uint4 *>(qs_dst) = make_uint4(w[0], w[1], w[2], w[3]);
    *d_dst = s16[0];
}

TG_DEV void planar_to_aos_block(const uint8_t *qs_src, const uint16_t *d_src, uint8_t *dst) {
    uint4 q = *reinterpret_cast<const uint4 *>(qs_src);
    uint16_t *d16 = reinterpret_cast<uint16_t *>(dst);
    uint32_t w[4] = {q.x, q.y, q.z, q.w};
    d16[0] = *d_src;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        d16[1 + 2 * k] = (uint16_t)(w[k] & 0xFFFFu);
        d16[2 + 2 * k] = (uint16_t)(w[k] >> 16);
    }
}

__global__ __launch_bounds__(256) void k_repack_layer(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                      Shape s, size_t nblocks, int to_planar) {
    size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= nblocks) return;
    size_t bpe = (size_t)2 * s.I * s.nbH + (size_t)s.H * s.nbI;
    int e = (int)(g / bpe);
    TensorRef t = locate_block(s, g - (size_t)e * bpe);
    size_t nt = (size_t)t.rows * t.nb;
    size_t tbase = (size_t)e * s.EB + t.off;
    if (to_planar) {
        aos_to_planar_block(src + tbase + t.local * Q40_BYTES, dst + tbase + t.local * 16,
                            reinterpret_cast<uint16_t *>(dst + tbase + nt * 16) + t.local);
    } else {
        planar_to_aos_block(src + tbase + t.local * 16,
                            reinterpret_cast<const uint16_t *>(src + tbase + nt * 16) + t.local,
                            dst + tbase + t.local * Q40_BYTES);
    }
}

__global__ __launch_bounds__(256) void k_repack_tensor(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                       size_t n, int to_planar) {
    size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n) return;
    if (to_planar)
        aos_to_planar_block(src + g * Q40_BYTES, dst + g * 16, reinterpret_cast<uint16_t *>(dst + n * 16) + g);
    else
        planar_to_aos_block(src + g * 16, reinterpret_cast<const uint16_t *>(src + n * 16) + g, dst + g * Q40_BYTES);
}

// ========================================================== Q8_0 pieces
// Quantize n values (n multiple of 32) into the LDS activation form: qs
// (int8, 32 per block), dsc (float(half d)) and sum (sum of the block's q).
// Called by every thread of a 256-thread block; 32-lane groups are whole
// blocks, so a group is on or off as a unit and the shuffles are uniform.
TG_DEV void q8_to_lds(const float *__restrict__ src, int n, int8_t *qs, float *dsc, int *sum,
                      float scale, bool apply_scale) {
    for (int base = 0; base < n; base += 256) {
        int i = base + (int)threadIdx.x;
        bool on = i < n;
        float v = on ? src[i] : 0.0f;
        if (apply_scale) v = v * scale;
        float dq; int qsum; uint16_t dh;
        int q = q8_lane(v, dq, qsum, dh);
        if (on) {
            qs[i] = (int8_t)q;
            if ((i & 31) == 0) { dsc[i >> 5] = dq; sum[i >> 5] = qsum; }
        }
    }
}

__global__ __launch_bounds__(256) void k_quantize_q8_0(const float *__restrict__ x, uint8_t *__restrict__ out, int n) {
    int i = blockIdx.x * 256 + threadIdx.x;
    bool on = i < n;
    float v = on ? x[i] : 0.0f;
    float dq; int qsum; uint16_t dh;
    int q = q8_lane(v, dq, qsum, dh);
    if (on) {
        uint8_t *blk = out + (size_t)(i >> 5) * Q80_BYTES;
        blk[2 + (i & 31)] = (uint8_t)(int8_t)q;
        if ((i & 31) == 0) {
            blk[0] = (uint8_t)(dh & 0xFF);
            blk[1] = (uint8_t)(dh >> 8);
        }
    }
}

// Q8_0 blocks (34 B, global) -> LDS activation form.
TG_DEV void q8blocks_to_lds(const uint8_t *__restrict__ xq8, int nb, int8_t *qs, float *dsc, int *sum) {
    for (int i = threadIdx.x; i < nb * QK; i += blockDim.x) {
        const uint8_t *blk = xq8 + (size_t)(i >> 5) * Q80_BYTES;
        qs[i] = (int8_t)blk[2 + (i & 31)];
    }
    for (int b = threadIdx.x; b < nb; b += blockDim.x) {
        const uint8_t *blk = xq8 + (size_t)b * Q80_BYTES;
        dsc[b] = h2f((uint16_t)(blk[0] | (blk[1] << 8)));
        int s = 0;
        for (int j = 0; j < QK; j++) s += (int8_t)blk[2 + j];
        sum[b] = s;
    }
}

// ===================================================== row-dot machinery
// Where row-dot rd of a tile reads: its planar nibble groups and scales
// (pointers already at the row) and its activation (LDS qs and sums).
struct RowSrc {
    const uint4 *q;
    const uint16_t *d;
    const int8_t *xq;
    const int *xs;
    bool valid;
};

// U[rd * ustride + b] = round(S_b * dw_b) for nrd row-dots of nb blocks.
// UNR (row, block) items per thread are loaded before any is used, so each
// thread keeps UNR 16-byte loads in flight.
template <int UNR, typename RowFn>
TG_DEV void tile_terms(int nrd, int nb, float *U, int ustride, RowFn rowfn) {
    const int items = nrd * nb;
    for (int base = 0; base < items; base += 256 * UNR) {
        uint4 wv[UNR];
        uint16_t dv[UNR];
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            int p = base + u * 256 + (int)threadIdx.x;
            wv[u] = make_uint4(0u, 0u, 0u, 0u);
            dv[u] = 0;
            if (p < items) {
                int rd = p / nb, b = p - rd * nb;
                RowSrc rs = rowfn(rd);
                if (rs.valid) {
                    wv[u] = rs.q[b];
                    dv[u] = rs.d[b];
                }
            }
        }
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            int p = base + u * 256 + (int)threadIdx.x;
            if (p < items) {
                int rd = p / nb, b = p - rd * nb;
                RowSrc rs = rowfn(rd);
                int sd = dot_q4_q8(wv[u], reinterpret_cast<const int *>(rs.xq + b * QK));
                int S = sd - 8 * rs.xs[b];
                U[rd * ustride + b] = (float)S * h2f(dv[u]);
            }
        }
    }
}

// Sequential per-row accumulation acc = fma(U_b, dx_b, acc).
TG_DEV float chain(const float *U, const float *dx, int nb) {
    float acc = 0.0f;
    for (int b = 0; b < nb; b++) acc = __builtin_fmaf(U[b], dx[b], acc);
    return acc;
}

// ============================================================ top-k
// Top-k of one token's E logits with renormalised softmax; one full wave.
// Selection: largest logit, equal logits -> lower expert index.  Softmax over
// the k values in ascending order with numpy's pairwise sum.  Results to LDS
// (sidx, sw; slog and sex are scratch).
TG_DEV void wave_topk(const float *__restrict__ logits, int E, int k, int *sidx, float *sw, float *slog,
                      float *sex) {
    const int lane = threadIdx.x & 63;
    constexpr int M = MAX_E / WAVE;
    float v[M];
    unsigned taken = 0;
#pragma unroll
    for (int m = 0; m < M; m++) {
        int e = lane + WAVE * m;
        v[m] = e < E ? logits[e] : 0.0f;
        if (e >= E) taken |= 1u << m;
    }
    for (int r = 0; r < k; r++) {
        float bv = -__builtin_inff();
        int bi = INT_MAX;
        bool have = false;
#pragma unroll
        for (int m = 0; m < M; m++) {
            if (!((taken >> m) & 1u) && (!have || v[m] > bv)) {
                bv = v[m];
                bi = lane + WAVE * m;
                have = true;
            }
        }
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) {
            float ov = __shfl_xor(bv, s, WAVE);
            int oi = __shfl_xor(bi, s, WAVE);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if ((bi & (WAVE - 1)) == lane) taken |= 1u << (bi / WAVE);
        if (lane == 0) { sidx[r] = bi; slog[r] = bv; }
    }
    if (lane == 0) {
        float lmax = slog[0];
        for (int i = 0; i < k; i++) sex[i] = expf_tg(slog[k - 1 - i] - lmax);
        float sum = np_pairwise_sum(sex, k);
        for (int i = 0; i < k; i++) sw[k - 1 - i] = sex[i] / sum;
    }
}

__global__ __launch_bounds__(64) void k_topk(const float *__restrict__ logits, int E, int k,
                                             int32_t *__restrict__ idx, float *__restrict__ w) {
    __shared__ int sidx[MAX_K];
    __shared__ float sw[MAX_K], slog[MAX_K], sex[MAX_K];
    const int t = blockIdx.x;
    wave_topk(logits + (size_t)t * E, E, k, sidx, sw, slog, sex);
    __syncthreads();
    if ((int)threadIdx.x < k) {
        if (idx) idx[(size_t)t * k + threadIdx.x] = sidx[threadIdx.x];
        if (w) w[(size_t)t * k + threadIdx.x] = sw[threadIdx.x];
    }
}

// ============================================================ router
// logits[t][e] = Wr[e] . (x[t] * s), s = 1/sqrt(mean(x^2) + eps).  Each wave
// takes one expert row: lane l fma-accumulates float4 chunks l, l+64, ...,
// then an xor butterfly.  4 rows per 256-thread block.
__global__ __launch_bounds__(256) void k_router(const float *__restrict__ Wr, const float *__restrict__ x,
                                                int E, int H, float eps, float *__restrict__ logits) {
    __shared__ float red[4];
    const int t = blockIdx.y;
    const float *xt = x + (size_t)t * H;
    float sc = rms_scale(block_sumsq(xt, H, red), H, eps);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int e = blockIdx.x * 4 + wave;
    if (e >= E) return;
    const float4 *w4 = reinterpret_cast<const float4 *>(Wr + (size_t)e * H);
    const float4 *x4 = reinterpret_cast<const float4 *>(xt);
    float acc = 0.0f;
    for (int q = lane; q < H / 4; q += WAVE) {
        float4 wv = w4[q], xv = x4[q];
        acc = __builtin_fmaf(wv.x, xv.x * sc, acc);
        acc = __builtin_fmaf(wv.y, xv.y * sc, acc);
        acc = __builtin_fmaf(wv.z, xv.z * sc, acc);
        acc = __builtin_fmaf(wv.w, xv.w * sc, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) logits[(size_t)t * E + e] = acc;
}

// ============================================================ gate / up
// Grid (I/RT, k, T).  Block (rt, j, t) computes rows [rt*RT, rt*RT+RT) of
// gate and up of token t's j-th expert, then h = SiLU(gate) * up.  Every
// block re-derives the token's top-k and Q8_0(x / rms(x)) itself (cheap,
// identical everywhere), so no block waits on another.
constexpr int GU_RT = 16;

__global__ __launch_bounds__(256) void k_gateup(const uint8_t *__restrict__ layer_pl, Shape s,
                                                const float *__restrict__ x, const float *__restrict__ logits,
                                                float eps, float *__restrict__ h, int32_t *__restrict__ idx_out,
                                                float *__restrict__ w_out) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int RT = GU_RT;
    const int nb = s.nbH, ust = nb + 1;
    int8_t *xq = reinterpret_cast<int8_t *>(smem);
    float *xd = reinterpret_cast<float *>(smem + s.H);
    int *xs = reinterpret_cast<int *>(xd + nb);
    float *U = reinterpret_cast<float *>(xs + nb);
    float *accs = U + 2 * RT * ust;
    int *sidx = reinterpret_cast<int *>(accs + 2 * RT);
    float *sw = reinterpret_cast<float *>(sidx + MAX_K);
    float *slog = sw + MAX_K;
    float *sex = slog + MAX_K;
    float *red = sex + MAX_K;

    const int t = blockIdx.z, j = blockIdx.y, r0 = blockIdx.x * RT;
    const float *xt = x + (size_t)t * s.H;
    if (threadIdx.x < WAVE) wave_topk(logits + (size_t)t * s.E, s.E, s.k, sidx, sw, slog, sex);
    float sc = rms_scale(block_sumsq(xt, s.H, red), s.H, eps);
    q8_to_lds(xt, s.H, xq, xd, xs, sc, true);
    __syncthreads();
    if (blockIdx.x == 0 && j == 0 && (int)threadIdx.x < s.k) {
        if (idx_out) idx_out[(size_t)t * s.k + threadIdx.x] = sidx[threadIdx.x];
        if (w_out) w_out[(size_t)t * s.k + threadIdx.x] = sw[threadIdx.x];
    }
    const uint8_t *ex = layer_pl + (size_t)sidx[j] * s.EB;
    const size_t ntb = (size_t)s.I * nb;
    const int I = s.I;
    tile_terms<8>(2 * RT, nb, U, ust, [&](int rd) {
        int mat = rd >= RT ? 1 : 0;
        int row = r0 + (rd - mat * RT);
        const uint8_t *tb = ex + (size_t)mat * s.GB;
        RowSrc rs;
        rs.valid = row < I;
        size_t ro = (size_t)(row < I ? row : 0) * nb;
        rs.q = reinterpret_cast<const uint4 *>(tb) + ro;
        rs.d = reinterpret_cast<const uint16_t *>(tb + ntb * 16) + ro;
        rs.xq = xq;
        rs.xs = xs;
        return rs;
    });
    __syncthreads();
    if ((int)threadIdx.x < 2 * RT) accs[threadIdx.x] = chain(U + threadIdx.x * ust, xd, nb);
    __syncthreads();
    if ((int)threadIdx.x < RT && r0 + (int)threadIdx.x < I)
        h[((size_t)t * s.k + j) * I + r0 + threadIdx.x] = silu_mul(accs[threadIdx.x], accs[RT + threadIdx.x]);
}

// ============================================================ down
// Grid (H/RD, T).  Block (rb, t) computes rows [rb*RD, rb*RD+RD) of down
// for all k experts of token t and combines them: out = sum_j w_j down_j in
// ascending logit order (j = k-1 .. 0), plus resid when given.
constexpr int DN_RD = 8;

__global__ __launch_bounds__(256) void k_down(const uint8_t *__restrict__ layer_pl, Shape s,
                                              const float *__restrict__ h, const int32_t *__restrict__ idx,
                                              const float *__restrict__ w, const float *resid, float *out) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int RD = DN_RD;
    const int k = s.k, nb = s.nbI, I = s.I, H = s.H, ust = nb + 1;
    int8_t *hq = reinterpret_cast<int8_t *>(smem);
    float *hd = reinterpret_cast<float *>(smem + (size_t)k * I);
    int *hs = reinterpret_cast<int *>(hd + k * nb);
    float *U = reinterpret_cast<float *>(hs + k * nb);
    float *D = U + k * RD * ust;
    int *sidx = reinterpret_cast<int *>(D + k * RD);
    float *sw = reinterpret_cast<float *>(sidx + MAX_K);

    const int t = blockIdx.y, r0 = blockIdx.x * RD;
    if ((int)threadIdx.x < k) {
        sidx[threadIdx.x] = idx[(size_t)t * k + threadIdx.x];
        sw[threadIdx.x] = w[(size_t)t * k + threadIdx.x];
    }
    q8_to_lds(h + (size_t)t * k * I, k * I, hq, hd, hs, 1.0f, false);
    __syncthreads();
    const size_t ntb = (size_t)H * nb;
    tile_terms<6>(k * RD, nb, U, ust, [&](int rd) {
        int jj = rd / RD;
        int row = r0 + (rd - jj * RD);
        const uint8_t *tb = layer_pl + (size_t)sidx[jj] * s.EB + 2 * s.GB;
        RowSrc rs;
        rs.valid = row < H;
        size_t ro = (size_t)(row < H ? row : 0) * nb;
        rs.q = reinterpret_cast<const uint4 *>(tb) + ro;
        rs.d = reinterpret_cast<const uint16_t *>(tb + ntb * 16) + ro;
        rs.xq = hq + (size_t)jj * I;
        rs.xs = hs + jj * nb;
        return rs;
    });
    __syncthreads();
    if ((int)threadIdx.x < k * RD) {
        int jj = threadIdx.x / RD;
        D[threadIdx.x] = chain(U + threadIdx.x * ust, hd + jj * nb, nb);
    }
    __syncthreads();
    if ((int)threadIdx.x < RD && r0 + (int)threadIdx.x < H) {
        float acc = 0.0f;
        for (int jj = k - 1; jj >= 0; jj--) acc = __builtin_fmaf(sw[jj], D[jj * RD + threadIdx.x], acc);
        size_t o = (size_t)t * H + r0 + threadIdx.x;
        out[o] = resid ? resid[o] + acc : acc;
    }
}

// ================================================ stand-alone row dots
// Exact block sums of a planar matrix against Q8_0 blocks (34 B).
__global__ __launch_bounds__(256) void k_block_sums(const uint8_t *__restrict__ w_pl, int rows, int nb,
                                                    const uint8_t *__restrict__ xq8, int32_t *__restrict__ sums) {
    size_t g = (size_t)blockIdx.x * 256 + threadIdx.x;
    size_t n = (size_t)rows * nb;
    if (g >= n) return;
    int b = (int)(g % (size_t)nb);
    uint4 wv = reinterpret_cast<const uint4 *>(w_pl)[g];
    const uint8_t *blk = xq8 + (size_t)b * Q80_BYTES;
    int x8[8];
    int xsum = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        uint32_t word = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            uint8_t byte = blk[2 + 4 * k + c];
            xsum += (int8_t)byte;
            word |= (uint32_t)byte << (8 * c);
        }
        x8[k] = (int)word;
    }
    sums[g] = dot_q4_q8(wv, x8) - 8 * xsum;
}

// out[r] = row r . x with the tile machinery (RT rows per block).
constexpr int MV_RT = 16;

__global__ __launch_bounds__(256) void k_matvec(const uint8_t *__restrict__ w_pl, int rows, int nb,
                                                const uint8_t *__restrict__ xq8, float *__restrict__ out) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int RT = MV_RT;
    const int ust = nb + 1;
    int8_t *xq = reinterpret_cast<int8_t *>(smem);
    float *xd = reinterpret_cast<float *>(smem + (size_t)nb * QK);
    int *xs = reinterpret_cast<int *>(xd + nb);
    float *U = reinterpret_cast<float *>(xs + nb);
    q8blocks_to_lds(xq8, nb, xq, xd, xs);
    __syncthreads();
    const int r0 = blockIdx.x * RT;
    const size_t ntb = (size_t)rows * nb;
    tile_terms<4>(RT, nb, U, ust, [&](int rd) {
        int row = r0 + rd;
        RowSrc rs;
        rs.valid = row < rows;
        size_t ro = (size_t)(row < rows ? row : 0) * nb;
        rs.q = reinterpret_cast<const uint4 *>(w_pl) + ro;
        rs.d = reinterpret_cast<const uint16_t *>(w_pl + ntb * 16) + ro;
        rs.xq = xq;
        rs.xs = xs;
        return rs;
    });
    __syncthreads();
    if ((int)threadIdx.x < RT && r0 + (int)threadIdx.x < rows)
        out[r0 + threadIdx.x] = chain(U + threadIdx.x * ust, xd, nb);
}

// ================================================================ launchers
static inline unsigned cdiv(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }

uint64_t host_stream_key(uint64_t seed, uint64_t stream) {
    auto mix = [](uint64_t x) {
        uint64_t z = x + 0x9E3779B97F4A7C15ull;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    };
    return mix(seed ^ mix(stream ^ 0x6A09E667F3BCC909ull));
}

hipError_t launch_synth_layer(uint8_t *layer_pl, float *router, const Shape &s, int layer, uint64_t seed,
                              float sigma, hipStream_t st) {
    size_t nblocks = (size_t)s.E * (2 * (size_t)s.I * s.nbH + (size_t)s.H * s.nbI);
    hipLaunchKernelGGL(k_synth_layer, dim3(cdiv(nblocks, 256)), dim3(256), 0, st, layer_pl, s, seed, layer,
                       sigma, nblocks);
    if (router) {
        size_t n = (size_t)s.E * s.H;
        hipLaunchKernelGGL(k_synth_normal, dim3(cdiv(n, 256)), dim3(256), 0, st, router,
                           host_stream_key(seed, stream_id(layer, 0, 3)), sigma, n);
    }
    return hipGetLastError();
}

hipError_t launch_synth_q40(uint8_t *pl, uint64_t key, float sigma, int rows, int nb, hipStream_t st) {
    size_t n = (size_t)rows * nb;
    hipLaunchKernelGGL(k_synth_q40, dim3(cdiv(n, 256)), dim3(256), 0, st, pl, key, sigma, rows, nb);
    return hipGetLastError();
}

hipError_t launch_synth_normal(float *out, uint64_t key, float sigma, size_t n, hipStream_t st) {
    hipLaunchKernelGGL(k_synth_normal, dim3(cdiv(n, 256)), dim3(256), 0, st, out, key, sigma, n);
    return hipGetLastError();
}

hipError_t launch_repack_layer(const uint8_t *src, uint8_t *dst, const Shape &s, bool to_planar, hipStream_t st) {
    size_t nblocks = (size_t)s.E * (2 * (size_t)s.I * s.nbH + (size_t)s.H * s.nbI);
    hipLaunchKernelGGL(k_repack_layer, dim3(cdiv(nblocks, 256)), dim3(256), 0, st, src, dst, s, nblocks,
                       to_planar ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_repack_tensor(const uint8_t *src, uint8_t *dst, size_t nblocks, bool to_planar, hipStream_t st) {
    hipLaunchKernelGGL(k_repack_tensor, dim3(cdiv(nblocks, 256)), dim3(256), 0, st, src, dst, nblocks,
                       to_planar ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_quantize_q8_0(const float *x, uint8_t *out, int n, hipStream_t st) {
    hipLaunchKernelGGL(k_quantize_q8_0, dim3(cdiv((size_t)n, 256)), dim3(256), 0, st, x, out, n);
    return hipGetLastError();
}

hipError_t launch_block_sums(const uint8_t *w_pl, int rows, int nb, const uint8_t *xq8, int32_t *sums,
                             hipStream_t st) {
    size_t n = (size_t)rows * nb;
    hipLaunchKernelGGL(k_block_sums, dim3(cdiv(n, 256)), dim3(256), 0, st, w_pl, rows, nb, xq8, sums);
    return hipGetLastError();
}

hipError_t launch_matvec(const uint8_t *w_pl, int rows, int nb, const uint8_t *xq8, float *out, hipStream_t st) {
    size_t lds = (size_t)nb * QK + 8 * (size_t)nb + 4 * (size_t)MV_RT * (nb + 1);
    hipLaunchKernelGGL(k_matvec, dim3(cdiv((size_t)rows, MV_RT)), dim3(256), lds, st, w_pl, rows, nb, xq8, out);
    return hipGetLastError();
}

hipError_t launch_router(const float *Wr, const float *x, int T, int E, int H, float eps, float *logits,
                         hipStream_t st) {
    hipLaunchKernelGGL(k_router, dim3(cdiv((size_t)E, 4), T), dim3(256), 0, st, Wr, x, E, H, eps, logits);
    return hipGetLastError();
}

hipError_t launch_topk(const float *logits, int T, int E, int k, int32_t *idx, float *w, hipStream_t st) {
    hipLaunchKernelGGL(k_topk, dim3(T), dim3(64), 0, st, logits, E, k, idx, w);
    return hipGetLastError();
}

hipError_t launch_gateup(const uint8_t *layer_pl, const Shape &s, const float *x, const float *logits, int T,
                         float eps, float *h, int32_t *idx, float *w, hipStream_t st) {
    size_t lds = (size_t)s.H + 8 * (size_t)s.nbH + 4 * (size_t)2 * GU_RT * (s.nbH + 1) + 4 * 2 * GU_RT +
                 4 * 4 * MAX_K + 16;
    hipLaunchKernelGGL(k_gateup, dim3(cdiv((size_t)s.I, GU_RT), s.k, T), dim3(256), lds, st, layer_pl, s, x,
                       logits, eps, h, idx, w);
    return hipGetLastError();
}

hipError_t launch_down(const uint8_t *layer_pl, const Shape &s, const float *h, const int32_t *idx, const float *w,
                       int T, const float *resid, float *out, hipStream_t st) {
    size_t lds = (size_t)s.k * s.I + 8 * (size_t)s.k * s.nbI + 4 * (size_t)s.k * DN_RD * (s.nbI + 1) +
                 4 * (size_t)s.k * DN_RD + 8 * MAX_K;
    hipLaunchKernelGGL(k_down, dim3(cdiv((size_t)s.H, DN_RD), T), dim3(256), lds, st, layer_pl, s, h, idx, w,
                       resid, out);
    return hipGetLastError();
}

}  // namespace tg
