// tg_legacy.hip -- the reference's legacy (Q4_K / Q6_K / f16 / f32) entry
// points on the GPU: the 256-element Q8 activation quantizer, the Q4_K and
// Q6_K row dots, the f16 / f32 matrix-vector products, the RMS norm and the
// pieces of the expert forward (csrc/libtinygiant.c:42-340, 555-741).
//
// Every kernel performs the reference's arithmetic step for step: integer
// dots are exact in any order, and every fp32 operation happens in the order
// and with the roundings of the reference's scalar definition (contraction
// off, correctly rounded division and square root), so results equal the CPU
// restatement bit for bit.  These are compatibility paths (the reference ABI
// hands over host pointers per call); the Q4_0 arena path is the fast one.
#include "tg_device.h"
#include "tg_internal.h"

namespace tg {

// q8_block of libtinygiant.c:55-59: per 256 activations an fp32 scale, the
// int32 sum of the quantized values and the 256 int8 values
struct Q8K {
    float scale;
    int32_t sum;
    int8_t qs[LG_QK];
};
static_assert(sizeof(Q8K) == LG_Q8K_BYTES, "q8_block layout");

TG_DEV uint16_t ld16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

TG_DEV int8_t byte_s8(uint32_t w, int i) { return (int8_t)(uint8_t)(w >> (8 * i)); }

// get_scale_min_k4, libtinygiant.c:42-51: the 6-bit scale and min of
// sub-block j from the 12-byte field s
TG_DEV void scale_min_k4(int j, const uint8_t *s, int &sc, int &m) {
    if (j < 4) {
        sc = s[j] & 63;
        m = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// ------------------------------------------------------------ quantize_q8
// quantize_q8, libtinygiant.c:61-89: amax over the block, scale = amax/127,
// q = RNE(x * (127/amax)), the int32 sum of q.  One wave per block, lane l
// taking values 4l .. 4l+3.
// one 256-value block by one wave, lane l holding values 4 l .. 4 l + 3
TG_DEV void q8k_block(const float (&v)[4], int lane, Q8K *__restrict__ ob) {
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float f = fabsf(v[i]);
        a = f > a ? f : a;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float y = __shfl_xor(a, o, WAVE);
        a = y > a ? y : a;
    }
    const float inv = a > 0.0f ? 127.0f / a : 0.0f;
    int s = 0;
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int q = (int)__builtin_rintf(v[i] * inv);
        s += q;
        packed |= (uint32_t)(uint8_t)(int8_t)q << (8 * i);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, WAVE);
    reinterpret_cast<uint32_t *>(ob->qs)[lane] = packed;
    if (lane == 0) {
        ob->scale = a / 127.0f;
        ob->sum = s;
    }
}

__global__ __launch_bounds__(256) void k_quantize_q8k(const float *__restrict__ x, Q8K *__restrict__ out, int nblocks) {
    const int lane = threadIdx.x & 63, b = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nblocks) return;  // uniform over the wave
    const float4 v4 = reinterpret_cast<const float4 *>(x + (size_t)b * LG_QK)[lane];
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    q8k_block(v, lane, out + b);
}

// --------------------------------------------------------------- Q4_K dot
// y[r] = dot_q4k_q8(row r, xq), libtinygiant.c:104-169: per block, for each
// group g the integer dots of the 32 low and 32 high nibbles with their
// activations and the activations' sums, turned into
// (d sc_l) dl - (dmin m_l) su_l and (d sc_h) dh - (dmin m_h) su_h; the eight
// differences added in group order, blocks added in order as scale * sum.
// A wave walks a sequence of blocks (the blocks of consecutive rows, or one
// row's blocks over several experts) 16 at a time, one lane per (block,
// group): lane l takes block 16 p + l / 4 of pass p and its group g = l % 4,
// i.e. the 32 weight bytes 32 g .. +31 (low nibbles against activations
// 64 g .. +31, high nibbles against 64 g + 32 .. +63) and the block's d, dmin
// and scale bytes.  The integer dots are four-byte dot products; a block's
// eight group differences are added in order by broadcasts within its quad of
// lanes, and the blocks' scale * sum terms are added in order from the
// lanes that hold them (the row values are wave-uniform).  Loads are plain
// 16-byte loads at any alignment.
struct Q4kGrp {
    uint32_t dm, s0, s1, s2;  // d | dmin << 16, scale bytes 0-3, 4-7, 8-11
    uint4 q0, q1;             // weight bytes 32 g .. +31
};
struct Q8kGrp {
    uint4 l0, l1, h0, h1;  // activations 64 g .. +31 and 64 g + 32 .. +63
    float xs;
};

TG_DEV uint4 ldu4(const void *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}

TG_DEV void q4k_grp_load(const uint8_t *__restrict__ bl, int g, Q4kGrp &W) {
    const uint4 h = ldu4(bl);
    W.dm = h.x;
    W.s0 = h.y;
    W.s1 = h.z;
    W.s2 = h.w;
    W.q0 = ldu4(bl + 16 + 32 * g);
    W.q1 = ldu4(bl + 32 + 32 * g);
}

TG_DEV void q8k_grp_load(const Q8K *__restrict__ xb, int g, Q8kGrp &X) {
    const int8_t *q = xb->qs + 64 * g;
    X.l0 = ldu4(q);
    X.l1 = ldu4(q + 16);
    X.h0 = ldu4(q + 32);
    X.h1 = ldu4(q + 48);
    X.xs = xb->scale;
}

TG_DEV int ubyte(uint32_t w, int i) { return (int)((w >> (8 * i)) & 0xFF); }

// get_scale_min_k4 on the scale field held as three words
TG_DEV void scale_min_k4w(int j, uint32_t s0, uint32_t s1, uint32_t s2, int &sc, int &m) {
    if (j < 4) {
        sc = ubyte(s0, j) & 63;
        m = ubyte(s1, j) & 63;
    } else {
        sc = (ubyte(s2, j - 4) & 0xF) | ((ubyte(s0, j - 4) >> 6) << 4);
        m = (ubyte(s2, j - 4) >> 4) | ((ubyte(s1, j - 4) >> 6) << 4);
    }
}

// lane g of the lane's quad, by DPP (quad_perm [g, g, g, g])
template <int G>
TG_DEV float quad_lane(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), G * 0x55, 0xF, 0xF, false));
}

TG_DEV float lane_f(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }

// scale * (block sum over its groups in order), in every lane of the quad
TG_DEV float q4k_grp_term(const Q4kGrp &W, const Q8kGrp &X, int g) {
    const uint32_t q[8] = {W.q0.x, W.q0.y, W.q0.z, W.q0.w, W.q1.x, W.q1.y, W.q1.z, W.q1.w};
    const uint32_t xl[8] = {X.l0.x, X.l0.y, X.l0.z, X.l0.w, X.l1.x, X.l1.y, X.l1.z, X.l1.w};
    const uint32_t xh[8] = {X.h0.x, X.h0.y, X.h0.z, X.h0.w, X.h1.x, X.h1.y, X.h1.z, X.h1.w};
    int dl = 0, dh = 0, sul = 0, suh = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        dl = __builtin_amdgcn_sdot4((int)(q[i] & 0x0F0F0F0Fu), (int)xl[i], dl, false);
        dh = __builtin_amdgcn_sdot4((int)((q[i] >> 4) & 0x0F0F0F0Fu), (int)xh[i], dh, false);
        sul = __builtin_amdgcn_sdot4(0x01010101, (int)xl[i], sul, false);
        suh = __builtin_amdgcn_sdot4(0x01010101, (int)xh[i], suh, false);
    }
    const float d = h2f((uint16_t)(W.dm & 0xFFFF)), dmin = h2f((uint16_t)(W.dm >> 16));
    int sl, ml, sh, mh;
    scale_min_k4w(2 * g, W.s0, W.s1, W.s2, sl, ml);
    scale_min_k4w(2 * g + 1, W.s0, W.s1, W.s2, sh, mh);
    const float tl = (d * (float)sl) * (float)dl, ul = (dmin * (float)ml) * (float)sul;
    const float th = (d * (float)sh) * (float)dh, uh = (dmin * (float)mh) * (float)suh;
    const float difl = tl - ul, difh = th - uh;
    float bs = 0.0f;
    bs = bs + quad_lane<0>(difl);
    bs = bs + quad_lane<0>(difh);
    bs = bs + quad_lane<1>(difl);
    bs = bs + quad_lane<1>(difh);
    bs = bs + quad_lane<2>(difl);
    bs = bs + quad_lane<2>(difh);
    bs = bs + quad_lane<3>(difl);
    bs = bs + quad_lane<3>(difh);
    return X.xs * bs;
}

// The Q4_K form of one lane's share of a block (sub = the lane's group)
struct Q4kFmt {
    static constexpr int BYTES = LG_Q4K_BYTES;
    using G = Q4kGrp;
    using X = Q8kGrp;
    TG_DEV static void load(const uint8_t *bl, const Q8K *xb, int sub, G &w, X &x) {
        q4k_grp_load(bl, sub, w);
        q8k_grp_load(xb, sub, x);
    }
    TG_DEV static float term(const G &w, const X &x, int sub) { return q4k_grp_term(w, x, sub); }
};

// The values of rows of bpr blocks each: nblk consecutive blocks from wb
// (starting at a row's first block) against the Q8 blocks of x at xb, xs
// bytes apart (global memory, or a padded copy in LDS); lane 0 stores the k-th row's
// value at out[k].  Two passes' loads at a time (block indices clamped to the
// last block; the clamped lanes' terms are never added).
template <class F>
TG_DEV void rows_seq(const uint8_t *__restrict__ wb, int nblk, const uint8_t *xb, int xs, int bpr, int lane,
                     float *__restrict__ out) {
    const int j4 = lane >> 2, sub = lane & 3;
    float cur = 0.0f;
    int b = 0, k = 0;  // wave-uniform: the block within its row, the row
    for (int p0 = 0; p0 < nblk; p0 += 32) {
        typename F::G W[2];
        typename F::X X[2];
#pragma unroll
        for (int pp = 0; pp < 2; pp++) {
            const int f = min(p0 + 16 * pp + j4, nblk - 1);
            F::load(wb + (size_t)f * F::BYTES, reinterpret_cast<const Q8K *>(xb + (size_t)(f % bpr) * xs), sub, W[pp],
                    X[pp]);
        }
#pragma unroll
        for (int pp = 0; pp < 2; pp++) {
            const float t = F::term(W[pp], X[pp], sub);
#pragma unroll
            for (int j = 0; j < 16; j++) {
                if (p0 + 16 * pp + j >= nblk) break;  // uniform
                cur = cur + lane_f(t, 4 * j);
                if (++b == bpr) {
                    if (lane == 0) out[k] = cur;
                    k++;
                    b = 0;
                    cur = 0.0f;
                }
            }
        }
    }
}

// rows per wave: a power of two up to 16, with at most 32 blocks per wave
// when a row has at most 16 (rows of no blocks: 16)
__host__ __device__ inline int q4k_rows_per_wave(int bpr) {
    int r = 1;
    while (r < 16 && 2 * r * bpr <= 32) r *= 2;
    return r;
}

// R rows per wave (a power of two, from the launcher)
__global__ __launch_bounds__(256) void k_matmul_q4k(const uint8_t *__restrict__ W, const Q8K *__restrict__ xq,
                                                    float *__restrict__ y, int nrows, int bpr, int R) {
    const int lane = threadIdx.x & 63;
    const int r0 = R * __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (r0 >= nrows) return;  // uniform over the wave
    if (bpr == 0) {  // rows of no blocks: the empty sum
        if (lane < min(R, nrows - r0)) y[r0 + lane] = 0.0f;
        return;
    }
    rows_seq<Q4kFmt>(W + (size_t)r0 * bpr * LG_Q4K_BYTES, min(R, nrows - r0) * bpr,
                     reinterpret_cast<const uint8_t *>(xq), (int)sizeof(Q8K), bpr, lane, y + r0);
}

// ------------------------------------------------ moe_forward, all experts
// The k experts of tg_moe_forward (libtinygiant.c:647-655) in three launches:
// the Q8 of x and every expert's gate and up rows, every expert's
// SiLU(gate) * up quantized to Q8 blocks, and every output row's down dots
// added over the experts in their order (the reference zeroes the output,
// then adds weight * down expert by expert: the same additions, in the same
// order, from the same zero).  One wave per row or block.
// The block first forms the Q8 blocks of x itself, in LDS at a stride of
// LG_XQ_LDS bytes from byte 8 (so that every qs array is 16-byte aligned);
// each wave quantizes every fourth block.
constexpr int LG_XQ_LDS = 272;
__global__ __launch_bounds__(256) void k_moe_gateup_q4k(const LgMoeOps P, const float *__restrict__ x,
                                                        float *__restrict__ gu, int n_exp, int inter, int bpr) {
    extern __shared__ __align__(16) uint8_t lsm[];
    uint8_t *xl = lsm + 8;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    for (int b = wv; b < bpr; b += 4) {
        const float4 v4 = reinterpret_cast<const float4 *>(x + (size_t)b * LG_QK)[lane];
        const float v[4] = {v4.x, v4.y, v4.z, v4.w};
        q8k_block(v, lane, reinterpret_cast<Q8K *>(xl + b * LG_XQ_LDS));
    }
    __syncthreads();
    // R rows per wave, all of one matrix (R is a power of two at most 16 and
    // inter a multiple of 256)
    const int R = q4k_rows_per_wave(bpr);
    const int r = R * __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + wv);
    if (r >= n_exp * 2 * inter) return;  // uniform over the wave
    const int e = r / (2 * inter), rem = r - e * 2 * inter, m = rem >= inter ? 1 : 0, i = rem - m * inter;
    const uint8_t *W = m ? P.up[e] : P.gate[e];
    rows_seq<Q4kFmt>(W + (size_t)i * bpr * LG_Q4K_BYTES, R * bpr, xl, LG_XQ_LDS, bpr, lane, gu + r);  // gu[e][m][i]
}

__global__ __launch_bounds__(256) void k_moe_silu_q8k(const float *__restrict__ gu, Q8K *__restrict__ hq, int n_exp,
                                                      int inter) {
    const int lane = threadIdx.x & 63, b = blockIdx.x * 4 + (threadIdx.x >> 6), nbh = inter / LG_QK;
    if (b >= n_exp * nbh) return;  // uniform over the wave
    const int e = b / nbh, j = b - e * nbh;
    const float *g = gu + (size_t)e * 2 * inter + (size_t)j * LG_QK + 4 * lane, *u = g + inter;
    const float4 g4 = *reinterpret_cast<const float4 *>(g), u4 = *reinterpret_cast<const float4 *>(u);
    const float v[4] = {silu_mul(g4.x, u4.x), silu_mul(g4.y, u4.y), silu_mul(g4.z, u4.z), silu_mul(g4.w, u4.w)};
    q8k_block(v, lane, hq + b);  // hq[e][j]
}

// the expert of lane-varying index e (< n) from the wave-uniform table
TG_DEV const uint8_t *pick_expert(const uint8_t *const (&t)[LG_MOE_MAX], int n, int e) {
    const uint8_t *p = t[0];
#pragma unroll
    for (int k = 1; k < LG_MOE_MAX; k++)
        if (k < n && e == k) p = t[k];
    return p;
}

// one output row per wave: the sequence of its n_exp * dbpr blocks (expert
// by expert), each expert's row value added as acc + w * value when its last
// block is in
// (acc starts at out[r] when add_to_out: expert_forward's out += w * down)
__global__ __launch_bounds__(256) void k_moe_down_acc_q4k(const LgMoeOps P, const Q8K *__restrict__ hq,
                                                          float *__restrict__ out, int n_exp, int embed, int dbpr,
                                                          int add_to_out) {
    const int lane = threadIdx.x & 63, r = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (r >= embed) return;  // uniform over the wave
    const int j4 = lane >> 2, g = lane & 3, nblk = n_exp * dbpr;
    float acc = add_to_out ? out[r] : 0.0f, cur = 0.0f;
    int b = 0, e = 0;  // wave-uniform: the block within the expert's row, the expert
    for (int p0 = 0; p0 < nblk; p0 += 32) {
        Q4kGrp W[2];
        Q8kGrp X[2];
#pragma unroll
        for (int pp = 0; pp < 2; pp++) {
            const int f = min(p0 + 16 * pp + j4, nblk - 1), fe = f / dbpr, fb = f - fe * dbpr;
            q4k_grp_load(pick_expert(P.down, n_exp, fe) + ((size_t)r * dbpr + fb) * LG_Q4K_BYTES, g, W[pp]);
            q8k_grp_load(hq + f, g, X[pp]);  // hq[e][fb]
        }
#pragma unroll
        for (int pp = 0; pp < 2; pp++) {
            const float t = q4k_grp_term(W[pp], X[pp], g);
#pragma unroll
            for (int j = 0; j < 16; j++) {
                if (p0 + 16 * pp + j >= nblk) break;  // uniform
                cur = cur + lane_f(t, 4 * j);
                if (++b == dbpr) {
                    acc = acc + P.w[e] * cur;
                    e++;
                    b = 0;
                    cur = 0.0f;
                }
            }
        }
    }
    if (lane == 0) out[r] = acc;
}

// --------------------------------------------------------------- Q6_K dot
// y[r] = dot_q6k_q8(row r, xq), libtinygiant.c:196-258: per block, for each
// half and each 16-element step `is` four integer dots d1..d4 of 6-bit
// values (low nibble | 2 high bits, minus 32) with activations 0, 32, 64 and
// 96 ahead; the sixteen products sc * d added in (half, is, 1..4) order;
// blocks added in order as (d * scale) * sum.  One lane per (block, step):
// lane l takes block l / 4 of its pass and (half, is) = (s / 2, s % 2) for
// s = l % 4, i.e. the step's 16 elements of each of the four dots; a value
// minus 32 times x is summed as the four-byte dot of the unsigned 6-bit
// values with x, minus 32 times the sum of x (the same integer).
struct Q6kGrp {
    uint4 l0, l1, h;  // ql[64 half + 16 is ..], ql[.. + 32], qh[32 half + 16 is ..]
    uint2 sc;         // scales 8 half .. +7
    uint32_t d;
};
struct Q8kStep {
    uint4 x1, x2, x3, x4;  // activations 128 half + 16 is + 0, 32, 64, 96 .. +15
    float xs;
};

struct Q6kFmt {
    static constexpr int BYTES = LG_Q6K_BYTES;
    using G = Q6kGrp;
    using X = Q8kStep;
    TG_DEV static void load(const uint8_t *bl, const Q8K *xb, int sub, G &w, X &x) {
        const int half = sub >> 1, is = sub & 1;
        w.l0 = ldu4(bl + half * 64 + is * 16);
        w.l1 = ldu4(bl + half * 64 + 32 + is * 16);
        w.h = ldu4(bl + 128 + half * 32 + is * 16);
        __builtin_memcpy(&w.sc, bl + 192 + half * 8, 8);
        w.d = ld16(bl + 208);
        const int8_t *q = xb->qs + half * 128 + is * 16;
        x.x1 = ldu4(q);
        x.x2 = ldu4(q + 32);
        x.x3 = ldu4(q + 64);
        x.x4 = ldu4(q + 96);
        x.xs = xb->scale;
    }
    // (d * x scale) * (the block's sixteen sc * dot products in order), in
    // every lane of the quad
    TG_DEV static float term(const G &w, const X &x, int sub) {
        const int is = sub & 1;
        const uint32_t L0[4] = {w.l0.x, w.l0.y, w.l0.z, w.l0.w}, L1[4] = {w.l1.x, w.l1.y, w.l1.z, w.l1.w};
        const uint32_t H[4] = {w.h.x, w.h.y, w.h.z, w.h.w};
        const uint32_t X1[4] = {x.x1.x, x.x1.y, x.x1.z, x.x1.w}, X2[4] = {x.x2.x, x.x2.y, x.x2.z, x.x2.w};
        const uint32_t X3[4] = {x.x3.x, x.x3.y, x.x3.z, x.x3.w}, X4[4] = {x.x4.x, x.x4.y, x.x4.z, x.x4.w};
        constexpr uint32_t M4 = 0x0F0F0F0Fu, M2 = 0x03030303u;
        constexpr int ONES = 0x01010101;
        int a1 = 0, a2 = 0, a3 = 0, a4 = 0, s1 = 0, s2 = 0, s3 = 0, s4 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q1 = (L0[i] & M4) | ((H[i] & M2) << 4);
            const uint32_t q2 = (L1[i] & M4) | (((H[i] >> 2) & M2) << 4);
            const uint32_t q3 = ((L0[i] >> 4) & M4) | (((H[i] >> 4) & M2) << 4);
            const uint32_t q4 = ((L1[i] >> 4) & M4) | (((H[i] >> 6) & M2) << 4);
            a1 = __builtin_amdgcn_sdot4((int)q1, (int)X1[i], a1, false);
            a2 = __builtin_amdgcn_sdot4((int)q2, (int)X2[i], a2, false);
            a3 = __builtin_amdgcn_sdot4((int)q3, (int)X3[i], a3, false);
            a4 = __builtin_amdgcn_sdot4((int)q4, (int)X4[i], a4, false);
            s1 = __builtin_amdgcn_sdot4(ONES, (int)X1[i], s1, false);
            s2 = __builtin_amdgcn_sdot4(ONES, (int)X2[i], s2, false);
            s3 = __builtin_amdgcn_sdot4(ONES, (int)X3[i], s3, false);
            s4 = __builtin_amdgcn_sdot4(ONES, (int)X4[i], s4, false);
        }
        const float t1 = (float)byte_s8(w.sc.x, is) * (float)(a1 - 32 * s1);
        const float t2 = (float)byte_s8(w.sc.x, is + 2) * (float)(a2 - 32 * s2);
        const float t3 = (float)byte_s8(w.sc.y, is) * (float)(a3 - 32 * s3);
        const float t4 = (float)byte_s8(w.sc.y, is + 2) * (float)(a4 - 32 * s4);
        float bs = 0.0f;
        bs = bs + quad_lane<0>(t1);
        bs = bs + quad_lane<0>(t2);
        bs = bs + quad_lane<0>(t3);
        bs = bs + quad_lane<0>(t4);
        bs = bs + quad_lane<1>(t1);
        bs = bs + quad_lane<1>(t2);
        bs = bs + quad_lane<1>(t3);
        bs = bs + quad_lane<1>(t4);
        bs = bs + quad_lane<2>(t1);
        bs = bs + quad_lane<2>(t2);
        bs = bs + quad_lane<2>(t3);
        bs = bs + quad_lane<2>(t4);
        bs = bs + quad_lane<3>(t1);
        bs = bs + quad_lane<3>(t2);
        bs = bs + quad_lane<3>(t3);
        bs = bs + quad_lane<3>(t4);
        return (h2f((uint16_t)(w.d & 0xFFFF)) * x.xs) * bs;
    }
};

// R rows per wave (a power of two, from the launcher)
__global__ __launch_bounds__(256) void k_matmul_q6k(const uint8_t *__restrict__ W, const Q8K *__restrict__ xq,
                                                    float *__restrict__ y, int nrows, int bpr, int R) {
    const int lane = threadIdx.x & 63;
    const int r0 = R * __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
    if (r0 >= nrows) return;  // uniform over the wave
    if (bpr == 0) {  // rows of no blocks: the empty sum
        if (lane < min(R, nrows - r0)) y[r0 + lane] = 0.0f;
        return;
    }
    rows_seq<Q6kFmt>(W + (size_t)r0 * bpr * LG_Q6K_BYTES, min(R, nrows - r0) * bpr,
                     reinterpret_cast<const uint8_t *>(xq), (int)sizeof(Q8K), bpr, lane, y + r0);
}

// ------------------------------------------------------ f16 / f32 matvec
// matvec_f16 / tg_f32_matvec, libtinygiant.c:277-318: eight fma chains over
// steps of 8 elements (chain c takes elements i + c), t_c = chain c + chain
// c + 4, sum = (t0 + t1) + (t2 + t3), then the tail (ncols % 8) one product
// and one add at a time.  Eight lanes per row (lane c carries chain c).
// x passes through LDS in chunks of MV_XS columns; each lane's weights are
// loaded MV_D steps at a time into two register sets taken in turn, so one
// set's loads are in flight while the other's fmas run.  Addresses are
// clamped into the row instead of branched around (a branch or select on a
// load makes the compiler wait for it in place); clamped steps are not added.
constexpr int MV_D = 16, MV_XS = 8192;

template <bool HALF>
__global__ __launch_bounds__(256) void k_matvec_two_acc(const void *__restrict__ A, const float *__restrict__ x,
                                                        float *__restrict__ y, int nrows, int ncols) {
    __shared__ float xs[MV_XS];
    const int tid = threadIdx.x, c = tid & 7, row = (blockIdx.x * 256 + tid) >> 3;
    const bool on = row < nrows;
    const int n8 = ncols & ~7;
    auto wat = [&](size_t i) -> float {
        return HALF ? h2f(reinterpret_cast<const uint16_t *>(A)[i]) : reinterpret_cast<const float *>(A)[i];
    };
    const size_t r0 = (size_t)(on ? row : nrows - 1) * ncols;
    float a = 0.0f;
    for (int x0 = 0; x0 < n8; x0 += MV_XS) {
        const int nx = min(MV_XS, n8 - x0), ns = nx >> 3;
        __syncthreads();  // the previous chunk of x is read
        for (int i0 = 0; i0 < nx; i0 += 256 * 8) {
            float t[8];
#pragma unroll
            for (int u = 0; u < 8; u++) t[u] = x[x0 + min(i0 + tid + 256 * u, nx - 1)];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = i0 + tid + 256 * u;
                if (i < nx) xs[i] = t[u];
            }
        }
        __syncthreads();
        const size_t wb = r0 + x0 + c;
        float pa[MV_D], pb[MV_D], xa[MV_D], xb[MV_D];
        auto ld = [&](float *p, float *q, int s0) {  // weights from HBM, x from LDS
#pragma unroll
            for (int k = 0; k < MV_D; k++) {
                const int sk = min(s0 + k, ns - 1);
                p[k] = wat(wb + 8 * (size_t)sk);
                q[k] = xs[8 * sk + c];
            }
        };
        auto run = [&](const float *p, const float *q) {
#pragma unroll
            for (int k = 0; k < MV_D; k++) a = __builtin_fmaf(p[k], q[k], a);
        };
        int st = 0;
        ld(pa, xa, 0);
        for (; st + 2 * MV_D <= ns; st += 2 * MV_D) {
            ld(pb, xb, st + MV_D);
            run(pa, xa);
            ld(pa, xa, st + 2 * MV_D);
            run(pb, xb);
        }
        // fewer than 2 MV_D steps remain: pa holds steps st.., pb the next MV_D
        ld(pb, xb, st + MV_D);
#pragma unroll
        for (int k = 0; k < MV_D; k++)
            if (st + k < ns) a = __builtin_fmaf(pa[k], xa[k], a);
#pragma unroll
        for (int k = 0; k < MV_D; k++)
            if (st + MV_D + k < ns) a = __builtin_fmaf(pb[k], xb[k], a);
    }
    const float t = a + __shfl_xor(a, 4, WAVE);  // lanes c < 4: chain c + chain c + 4
    const float t1 = __shfl_xor(t, 1, WAVE);
    const float u = t + t1;                      // lane 0: t0 + t1, lane 2: t2 + t3
    const float u2 = __shfl_xor(u, 2, WAVE);
    if (on && c == 0) {
        float sum = u + u2;
        for (int i = n8; i < ncols; i++) sum = sum + wat(r0 + i) * x[i];
        y[row] = sum;
    }
}

// --------------------------------------------------------------- RMS norm
// tg_rms_norm, libtinygiant.c:322-340: four fma chains of squares over
// steps of 4, ss = (v0 + v1) + (v2 + v3), the tail one product and add at a
// time, scale = 1 / sqrt(ss / dim + eps), out = (x * scale) * w.  One block
// per row (row b at x + b * dim, the same weight w).  The row passes
// through LDS in chunks of 4096 values, loaded by all threads with their
// loads in flight together, so the four chains (threads 0-3) read LDS
// rather than wait on a global load per step.
constexpr int RMS_CH = 4096;

__global__ __launch_bounds__(256) void k_rms_norm(const float *__restrict__ x, const float *__restrict__ w,
                                                  float *__restrict__ out, int dim, float eps) {
    __shared__ float xs[RMS_CH];
    __shared__ float v[4];
    __shared__ float scale;
    const int tid = threadIdx.x, n4 = dim & ~3;
    x += (size_t)blockIdx.x * dim;
    out += (size_t)blockIdx.x * dim;
    float a = 0.0f;
    for (int c0 = 0; c0 < n4; c0 += RMS_CH) {
        const int n = min(RMS_CH, n4 - c0);
        float xv[RMS_CH / 256];
#pragma unroll
        for (int u = 0; u < RMS_CH / 256; u++) xv[u] = x[c0 + min(tid + 256 * u, n - 1)];
        __syncthreads();  // the previous chunk is read
#pragma unroll
        for (int u = 0; u < RMS_CH / 256; u++) xs[tid + 256 * u] = xv[u];
        __syncthreads();
        if (tid < 4) {
#pragma unroll 8
            for (int i = tid; i < n; i += 4) a = __builtin_fmaf(xs[i], xs[i], a);
        }
    }
    if (tid < 4) v[tid] = a;
    __syncthreads();
    if (tid == 0) {
        float ss = (v[0] + v[1]) + (v[2] + v[3]);
        for (int i = n4; i < dim; i++) ss = ss + x[i] * x[i];
        scale = 1.0f / __builtin_sqrtf(ss / (float)dim + eps);
    }
    __syncthreads();
    const float sc = scale;
    for (int i = tid; i < dim; i += 256) out[i] = (x[i] * sc) * w[i];
}

// ------------------------------------------------ Q4_K, dequantize-then-dot
// tg_matmul_q4k_scalar, libtinygiant.c:706-741: every weight dequantized as
// (d sc) q - dmin m and the products with the fp32 input added pair by pair
// (low then high nibble) into one running total.  One thread per row.
__global__ __launch_bounds__(256) void k_matmul_q4k_scalar(const uint8_t *__restrict__ W, const float *__restrict__ x,
                                                           float *__restrict__ y, int nrows, int bpr) {
    const int row = blockIdx.x * 256 + threadIdx.x;
    if (row >= nrows) return;
    const uint8_t *wr = W + (size_t)row * bpr * LG_Q4K_BYTES;
    float total = 0.0f;
    for (int b = 0; b < bpr; b++) {
        const uint8_t *bl = wr + (size_t)b * LG_Q4K_BYTES;
        const float d = h2f(ld16(bl)), dmin = h2f(ld16(bl + 2));
        const uint8_t *qs = bl + 16;
        const float *xb = x + (size_t)b * LG_QK;
        for (int g = 0; g < 4; g++) {
            int sl, ml, sh, mh;
            scale_min_k4(2 * g, bl + 4, sl, ml);
            scale_min_k4(2 * g + 1, bl + 4, sh, mh);
            const float dsl = d * (float)sl, dsh = d * (float)sh, mml = dmin * (float)ml, mmh = dmin * (float)mh;
            for (int j = 0; j < 32; j++) {
                const int v = qs[g * 32 + j];
                const float vl = dsl * (float)(v & 0xF) - mml;
                const float vh = dsh * (float)(v >> 4) - mmh;
                total = total + (vl * xb[g * 64 + j] + vh * xb[g * 64 + 32 + j]);
            }
        }
    }
    y[row] = total;
}

// ------------------------------------------------------ expert forward bits
// hidden = SiLU(gate) * up (libtinygiant.c:580-583)
__global__ __launch_bounds__(256) void k_silu_mul_vec(const float *__restrict__ g, const float *__restrict__ u,
                                                      float *__restrict__ h, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) h[i] = silu_mul(g[i], u[i]);
}

// output[i] += weight * down[i] (libtinygiant.c:593-594): product, then add
__global__ __launch_bounds__(256) void k_acc_scaled(float *__restrict__ out, const float *__restrict__ v, float w,
                                                    int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = out[i] + w * v[i];
}

// -------------------------------------------------------------- attention
// apply_rope_inplace, libtinygiant.c:344-361, at one position (c, s: the
// tables' row): x1' = x1 c - x2 s (products rounded, then the difference:
// vmlsq_f32), x2' = fma(x1, s, x2 c) (vfmaq_f32 on the rounded x2 c).  One
// thread per pair (head h, i < half).
__global__ __launch_bounds__(256) void k_rope(float *__restrict__ x, int n_heads, int hd, const float *__restrict__ c,
                                              const float *__restrict__ sn) {
    const int half = hd / 2, p = blockIdx.x * 256 + threadIdx.x;
    if (p >= n_heads * half) return;
    const int h = p / half, i = p - h * half;
    float *xh = x + (size_t)h * hd;
    const float x1 = xh[i], x2 = xh[half + i];
    const float a = x1 * c[i], b = x2 * sn[i];
    xh[i] = a - b;
    xh[half + i] = __builtin_fmaf(x1, sn[i], x2 * c[i]);
}

// The new key and value rows into the caches [n_kv][seq][hd] at row `row`
// (libtinygiant.c:395-401).
__global__ __launch_bounds__(256) void k_kv_append(const float *__restrict__ kn, const float *__restrict__ v,
                                                   float *__restrict__ kc, float *__restrict__ vc, int n_kv, int seq,
                                                   int hd, int row) {
    const int p = blockIdx.x * 256 + threadIdx.x;
    if (p >= n_kv * hd) return;
    const int h = p / hd, d = p - h * hd;
    kc[((size_t)h * seq + row) * hd + d] = kn[p];
    vc[((size_t)h * seq + row) * hd + d] = v[p];
}

// Attention over seq cached positions (libtinygiant.c:405-446), the head's
// arithmetic in the reference's order: score_t = dot(q, k_t) * inv_sqrt, the
// dot in four fma lanes over steps of 4 added as (l0 + l1) + (l2 + l3) with
// the tail one product and add at a time; e_t = exp(score_t - max); sum =
// e_0 + e_1 + ... in order; out[d] = fma chain over t of (e_t * (1 / sum))
// v_t[d] (the tail d unfused).  The scores and the max are free of order,
// the two sums are not: the first launch spreads the dots over (kv head,
// 16 positions) blocks that share the K rows among the kv head's query heads;
// the second gives each (head group, 16 elements of d) block the sequential
// sums, with the V slice shared by the group's heads.
//
// A group is up to ATT_HB query heads of one kv head: group hg of kv head
// g = hg / ngrp starts at head g * ratio + (hg % ngrp) * ATT_HB.
TG_DEV void att_group(int hg, int ratio, int ngrp, int &g, int &h0, int &nh) {
    g = hg / ngrp;
    const int sub = hg - g * ngrp;
    h0 = g * ratio + sub * ATT_HB;
    nh = min(ATT_HB, ratio - sub * ATT_HB);
}

// n rows of hd floats (contiguous at src) into LDS rows of `stride` floats:
// every thread's loads of a round are in flight together (16 float4 when hd
// is a multiple of 4, else 16 floats), then stored.  256 threads.
TG_DEV void att_stage(float *dst, int stride, const float *__restrict__ src, int n, int hd) {
    const int tid = threadIdx.x, total = n * hd;
    if ((hd & 3) == 0) {
        const float4 *s4 = reinterpret_cast<const float4 *>(src);
        const int t4 = total >> 2, h4 = hd >> 2;
        for (int base = 0; base < t4; base += 256 * 16) {
            float4 v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const int i = base + u * 256 + tid;
                v[u] = i < t4 ? s4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const int i = base + u * 256 + tid;
                if (i < t4) {
                    const int rr = i / h4, c = 4 * (i - rr * h4);
                    float *o = dst + rr * stride + c;
                    o[0] = v[u].x; o[1] = v[u].y; o[2] = v[u].z; o[3] = v[u].w;
                }
            }
        }
    } else {
        for (int base = 0; base < total; base += 256 * 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const int i = base + u * 256 + tid;
                v[u] = i < total ? src[i] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const int i = base + u * 256 + tid;
                if (i < total) {
                    const int rr = i / hd;
                    dst[rr * stride + i - rr * hd] = v[u];
                }
            }
        }
    }
}

// Scores of one group's heads at positions [16 blockIdx.x, +16): a thread
// pair per (head, position), lanes 0-1 and 2-3 of the dot, K rows padded to
// hd + 1 floats in LDS.  scr: [n_heads][seq] scores, then [n_heads][nblk]
// maxima of each block's scores (starting from -1e30 and passing over NaN,
// as the reference's running max does).
template <bool VEC>  // VEC: hd % 4 == 0, q and K rows loaded as float4 in one round
__global__ __launch_bounds__(256) void k_attn_scores(const float *__restrict__ q, const float *__restrict__ kc,
                                                     float *__restrict__ scr, int n_heads, int seq, int hd, int ratio,
                                                     int ngrp, float inv_sqrt) {
    extern __shared__ __align__(16) float lds[];  // [ATT_HB][hd] q rows, then [ATT_TP][hd + 1] K rows
    int g, h0, nh;
    att_group(blockIdx.y, ratio, ngrp, g, h0, nh);
    const int tid = threadIdx.x, t0 = blockIdx.x * ATT_TP, n = min(ATT_TP, seq - t0), ks = hd + 1, hd4 = hd & ~3;
    float *qs = lds, *kr = lds + ATT_HB * hd;
    const float *qg = q + (size_t)h0 * hd, *kg = kc + ((size_t)g * seq + t0) * hd;
    if constexpr (VEC) {
        // hd <= 512: at most 4 float4 of q and 8 of K per thread, all in flight
        // (addresses clamped into the rows, not branched around)
        const int h4 = hd >> 2, nq = nh * h4, nk = n * h4;
        float4 qv[4], kv[8];
#pragma unroll
        for (int u = 0; u < 4; u++) qv[u] = reinterpret_cast<const float4 *>(qg)[min(tid + 256 * u, nq - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++) kv[u] = reinterpret_cast<const float4 *>(kg)[min(tid + 256 * u, nk - 1)];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = tid + 256 * u;
            if (i < nq) reinterpret_cast<float4 *>(qs)[i] = qv[u];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = tid + 256 * u;
            if (i < nk) {
                const int rr = i / h4, c = 4 * (i - rr * h4);
                float *o = kr + rr * ks + c;
                o[0] = kv[u].x; o[1] = kv[u].y; o[2] = kv[u].z; o[3] = kv[u].w;
            }
        }
    } else {
        att_stage(qs, hd, qg, nh, hd);
        att_stage(kr, ks, kg, n, hd);
    }
    __syncthreads();
    const int j = tid >> 1, hf = tid & 1, hl = j / ATT_TP, p = j - hl * ATT_TP;
    const bool ok = hl < nh && p < n;
    const float *qh = qs + hl * hd, *kt = kr + p * ks;
    float a0 = 0.0f, a1 = 0.0f;
    if (ok) {
#pragma unroll 8
        for (int d = 2 * hf; d < hd4; d += 4) {
            a0 = __builtin_fmaf(qh[d], kt[d], a0);
            a1 = __builtin_fmaf(qh[d + 1], kt[d + 1], a1);
        }
    }
    const float mine = a0 + a1, other = __shfl_xor(mine, 1, WAVE);
    float m = -1e30f;
    if (ok && hf == 0) {
        float dot = mine + other;  // (l0 + l1) + (l2 + l3)
        for (int d = hd4; d < hd; d++) dot = dot + qh[d] * kt[d];
        const float sv = dot * inv_sqrt;
        scr[(size_t)(h0 + hl) * seq + t0 + p] = sv;
        m = sv > m ? sv : m;
    }
    // a head's 16 positions are 32 consecutive lanes
#pragma unroll
    for (int s = 1; s < 32; s <<= 1) {
        const float o = __shfl_xor(m, s, WAVE);
        m = o > m ? o : m;
    }
    if ((tid & 31) == 0 && hl < nh)
        scr[(size_t)n_heads * seq + (size_t)(h0 + hl) * gridDim.x + blockIdx.x] = m;
}

// Softmax weights of one head (blockIdx.x): max over the scores blocks'
// maxima, e_t = exp(score_t - max), sum = e_0 + e_1 + ... in order (one
// lane's add chain through LDS, the next 16 values read while 16 are added),
// w_t = e_t * (1 / sum) into the weights rows.  Positions go through LDS in
// chunks of ATT_SC; with a single chunk the e_t stay there for the weights.
constexpr int ATT_SC = 2048;

__global__ __launch_bounds__(256) void k_attn_softmax(float *__restrict__ scr, int n_heads, int seq, int nblk,
                                                      size_t woff) {
    __shared__ __align__(16) float e[ATT_SC];
    __shared__ float red[4];
    __shared__ float bc;
    const int h = blockIdx.x, tid = threadIdx.x;
    const float *sc = scr + (size_t)h * seq;
    const float *pm = scr + (size_t)n_heads * seq + (size_t)h * nblk;
    float *w = scr + woff + (size_t)h * ((seq + 3) & ~3);
    constexpr int SU = ATT_SC / 256;
    float v[SU];
    // the first chunk's scores, then the maxima: all in flight together
#pragma unroll
    for (int u = 0; u < SU; u++) v[u] = sc[min(tid + 256 * u, seq - 1)];
    float mx = -1e30f;
    for (int b = tid; b < nblk; b += 256) {
        const float p = pm[b];
        mx = p > mx ? p : mx;
    }
#pragma unroll
    for (int s = 1; s < WAVE; s <<= 1) {
        const float o = __shfl_xor(mx, s, WAVE);
        mx = o > mx ? o : mx;
    }
    if ((tid & (WAVE - 1)) == 0) red[tid / WAVE] = mx;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; i++) mx = red[i] > mx ? red[i] : mx;
    float sum = 0.0f;
    for (int t0 = 0; t0 < seq; t0 += ATT_SC) {
        const int n = min(ATT_SC, seq - t0);
        if (t0 > 0) {
            __syncthreads();  // the previous chunk is summed
#pragma unroll
            for (int u = 0; u < SU; u++) v[u] = sc[min(t0 + tid + 256 * u, seq - 1)];
        }
#pragma unroll
        for (int u = 0; u < SU; u++) {
            const int i = tid + 256 * u;
            if (i < n) e[i] = expf_tg(v[u] - mx);
        }
        __syncthreads();
        if (tid == 0) {
            // 16 values a step in two register sets taken in turn: one set's
            // reads are in flight while the other's values are added
            const float4 *e4 = reinterpret_cast<const float4 *>(e);
            const int n16 = n >> 4;
            float4 a[4], b[4];
#pragma unroll
            for (int k = 0; k < 4; k++) a[k] = e4[k];
            int s16 = 0;
            for (; s16 + 2 <= n16; s16 += 2) {
#pragma unroll
                for (int k = 0; k < 4; k++) b[k] = e4[4 * (s16 + 1) + k];
#pragma unroll
                for (int k = 0; k < 4; k++) sum = ((sum + a[k].x) + a[k].y + a[k].z) + a[k].w;
                const int nx = 4 * min(s16 + 2, n16 - 1);
#pragma unroll
                for (int k = 0; k < 4; k++) a[k] = e4[nx + k];
#pragma unroll
                for (int k = 0; k < 4; k++) sum = ((sum + b[k].x) + b[k].y + b[k].z) + b[k].w;
            }
            if (s16 < n16) {
#pragma unroll
                for (int k = 0; k < 4; k++) sum = ((sum + a[k].x) + a[k].y + a[k].z) + a[k].w;
            }
            for (int i = 16 * n16; i < n; i++) sum = sum + e[i];
            bc = 1.0f / sum;
        }
    }
    __syncthreads();
    const float is = bc;
    if (seq <= ATT_SC) {
        for (int i = tid; i < seq; i += 256) w[i] = e[i] * is;
    } else {
        for (int i = tid; i < seq; i += 256) w[i] = expf_tg(sc[i] - mx) * is;
    }
}

// Weighted sum of one group's heads for d in [16 blockIdx.x, +16): thread
// (hl = tid / 16, r = tid % 16) carries out[h0 + hl][d0 + r] as one fma
// chain over the positions.  Weights and the V slice go through LDS in
// chunks of ATT_CH positions, the next chunk loaded into registers while the
// current one is summed; the LDS reads of the chain run 8 positions ahead.
constexpr int ATT_DS = 16, ATT_CH = 512, ATT_VU = ATT_CH * ATT_DS / 4 / 128, ATT_WU = ATT_HB * ATT_CH / 4 / 128;

template <bool VEC>  // VEC: hd % 4 == 0, the V slice read as float4
__global__ __launch_bounds__(128) void k_attn_wv(const float *__restrict__ scr, const float *__restrict__ vc,
                                                 float *__restrict__ out, int seq, int hd, int ratio, int ngrp,
                                                 size_t woff) {
    __shared__ __align__(16) float wl[ATT_HB][ATT_CH + 4];  // rows 16-byte aligned, 4 banks apart
    __shared__ __align__(16) float vs[ATT_CH * ATT_DS];
    int g, h0, nh;
    att_group(blockIdx.y, ratio, ngrp, g, h0, nh);
    const int tid = threadIdx.x, hl = tid >> 4, r = tid & 15, d0 = blockIdx.x * ATT_DS, hd4 = hd & ~3;
    const int seq4 = (seq + 3) & ~3;
    const float *wg = scr + woff + (size_t)h0 * seq4;
    const float *vg = vc + (size_t)g * seq * hd;
    float4 vr[ATT_VU], wr[ATT_WU];
    // Loads without branches or selects (either makes the compiler wait for
    // the load where it stands): each address is clamped into its buffer.  A
    // clamped position (t >= seq), element (d >= hd) or head (>= nh) holds a
    // copy of a valid value that no chain reads and no output stores.
    auto load = [&](int t0) {
        t0 = min(t0, seq - 1);  // a prefetch past the end reads the last chunk again
        const int n = min(ATT_CH, seq - t0);
#pragma unroll
        for (int u = 0; u < ATT_VU; u++) {
            const int i = tid + 128 * u, row = min(i >> 2, n - 1), c = d0 + 4 * (i & 3);
            const float *src = vg + (size_t)(t0 + row) * hd;
            if constexpr (VEC) {
                const float4 v = *reinterpret_cast<const float4 *>(src + min(c, hd - 4));
                vr[u].x = v.x;  // by component: a whole-float4 copy keeps the array out of registers
                vr[u].y = v.y;
                vr[u].z = v.z;
                vr[u].w = v.w;
            } else {
                vr[u].x = src[min(c, hd - 1)];
                vr[u].y = src[min(c + 1, hd - 1)];
                vr[u].z = src[min(c + 2, hd - 1)];
                vr[u].w = src[min(c + 3, hd - 1)];
            }
        }
#pragma unroll
        for (int u = 0; u < ATT_WU; u++) {
            const int i = tid + 128 * u, row = min(i / (ATT_CH / 4), nh - 1);
            const int p = min(t0 + 4 * (i & (ATT_CH / 4 - 1)), seq4 - 4);
            const float4 v = *reinterpret_cast<const float4 *>(wg + (size_t)row * seq4 + p);
            wr[u].x = v.x;
            wr[u].y = v.y;
            wr[u].z = v.z;
            wr[u].w = v.w;
        }
    };
    load(0);
    const int d = d0 + r;
    float o = 0.0f;
    for (int t0 = 0; t0 < seq; t0 += ATT_CH) {
        const int n = min(ATT_CH, seq - t0);
        lds_barrier();  // the previous chunk is consumed
#pragma unroll
        for (int u = 0; u < ATT_VU; u++)
            *reinterpret_cast<float4 *>(vs + 4 * (tid + 128 * u)) = make_float4(vr[u].x, vr[u].y, vr[u].z, vr[u].w);
#pragma unroll
        for (int u = 0; u < ATT_WU; u++) {
            const int i = tid + 128 * u;
            *reinterpret_cast<float4 *>(&wl[i / (ATT_CH / 4)][4 * (i & (ATT_CH / 4 - 1))]) =
                make_float4(wr[u].x, wr[u].y, wr[u].z, wr[u].w);
        }
        load(t0 + ATT_CH);  // past the end: harmless reloads, no branch
        lds_barrier();
        const float *w = wl[hl];
        if (d < hd4) {
            // 8 positions a step in two register sets taken in turn: one
            // set's LDS reads are in flight while the other's fmas run
            const float4 *w4 = reinterpret_cast<const float4 *>(w);
            const float *v = vs + r;
            const int n8 = n >> 3;
            float4 wa0, wa1, wb0, wb1;
            float va[8], vb[8];
            wa0 = w4[0]; wa1 = w4[1];
#pragma unroll
            for (int k = 0; k < 8; k++) va[k] = v[k * ATT_DS];
            int s8 = 0;
            for (; s8 + 2 <= n8; s8 += 2) {
                const int nb = 8 * (s8 + 1);
                wb0 = w4[nb >> 2]; wb1 = w4[(nb >> 2) + 1];
#pragma unroll
                for (int k = 0; k < 8; k++) vb[k] = v[(nb + k) * ATT_DS];
                o = __builtin_fmaf(wa0.x, va[0], o); o = __builtin_fmaf(wa0.y, va[1], o);
                o = __builtin_fmaf(wa0.z, va[2], o); o = __builtin_fmaf(wa0.w, va[3], o);
                o = __builtin_fmaf(wa1.x, va[4], o); o = __builtin_fmaf(wa1.y, va[5], o);
                o = __builtin_fmaf(wa1.z, va[6], o); o = __builtin_fmaf(wa1.w, va[7], o);
                const int na = 8 * min(s8 + 2, n8 - 1);
                wa0 = w4[na >> 2]; wa1 = w4[(na >> 2) + 1];
#pragma unroll
                for (int k = 0; k < 8; k++) va[k] = v[(na + k) * ATT_DS];
                o = __builtin_fmaf(wb0.x, vb[0], o); o = __builtin_fmaf(wb0.y, vb[1], o);
                o = __builtin_fmaf(wb0.z, vb[2], o); o = __builtin_fmaf(wb0.w, vb[3], o);
                o = __builtin_fmaf(wb1.x, vb[4], o); o = __builtin_fmaf(wb1.y, vb[5], o);
                o = __builtin_fmaf(wb1.z, vb[6], o); o = __builtin_fmaf(wb1.w, vb[7], o);
            }
            if (s8 < n8) {
                o = __builtin_fmaf(wa0.x, va[0], o); o = __builtin_fmaf(wa0.y, va[1], o);
                o = __builtin_fmaf(wa0.z, va[2], o); o = __builtin_fmaf(wa0.w, va[3], o);
                o = __builtin_fmaf(wa1.x, va[4], o); o = __builtin_fmaf(wa1.y, va[5], o);
                o = __builtin_fmaf(wa1.z, va[6], o); o = __builtin_fmaf(wa1.w, va[7], o);
            }
            for (int t = 8 * n8; t < n; t++) o = __builtin_fmaf(w[t], vs[t * ATT_DS + r], o);
        } else if (d < hd) {
            for (int t = 0; t < n; t++) o = o + w[t] * vs[t * ATT_DS + r];
        }
    }
    if (hl < nh && d < hd) out[(size_t)(h0 + hl) * hd + d] = o;
}

// x[i] += a[i] (libtinygiant.c:682,700)
__global__ __launch_bounds__(256) void k_add_vec(float *__restrict__ x, const float *__restrict__ a, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = x[i] + a[i];
}

// ----------------------------------------------------------------- argmax
// Greedy next token (engine.py:359, np.argmax): the first index of the
// largest value, NaN above every number (numpy returns the first NaN).
// Blocks reduce grid-strided slices to (value, index) partials; one block
// reduces the partials in index order of the slices.
TG_DEV bool am_better(float av, int ai, float bv, int bi) {
    const bool an = av != av, bn = bv != bv;
    if (an || bn) return an && (!bn || ai < bi);
    return av > bv || (av == bv && ai < bi);
}

TG_DEV void am_block(float &v, int &i) {
    __shared__ float sv[256 / WAVE];
    __shared__ int si[256 / WAVE];
#pragma unroll
    for (int s = 1; s < WAVE; s <<= 1) {
        const float ov = __shfl_xor(v, s, WAVE);
        const int oi = __shfl_xor(i, s, WAVE);
        if (am_better(ov, oi, v, i)) { v = ov; i = oi; }
    }
    const int tid = threadIdx.x;
    if ((tid & (WAVE - 1)) == 0) { sv[tid / WAVE] = v; si[tid / WAVE] = i; }
    __syncthreads();
    v = sv[0]; i = si[0];
#pragma unroll
    for (int w = 1; w < 256 / WAVE; w++)
        if (am_better(sv[w], si[w], v, i)) { v = sv[w]; i = si[w]; }
}

__global__ __launch_bounds__(256) void k_argmax_part(const float *__restrict__ x, int n, float *__restrict__ pv,
                                                     int *__restrict__ pi) {
    float v = x[0];
    int i = 0;
    for (int j = blockIdx.x * 256 + threadIdx.x; j < n; j += gridDim.x * 256) {
        const float xv = x[j];
        if (am_better(xv, j, v, i)) { v = xv; i = j; }
    }
    am_block(v, i);
    if (threadIdx.x == 0) { pv[blockIdx.x] = v; pi[blockIdx.x] = i; }
}

__global__ __launch_bounds__(256) void k_argmax_final(const float *__restrict__ pv, const int *__restrict__ pi, int nb,
                                                      int *__restrict__ out) {
    float v = pv[0];
    int i = pi[0];
    for (int b = threadIdx.x; b < nb; b += 256)
        if (am_better(pv[b], pi[b], v, i)) { v = pv[b]; i = pi[b]; }
    am_block(v, i);
    if (threadIdx.x == 0) out[0] = i;
}

// ------------------------------------------------------------- launchers
static unsigned lg_cdiv(long n, long d) { return (unsigned)((n + d - 1) / d); }

hipError_t launch_quantize_q8k(const float *x, void *xq, int nblocks, hipStream_t st) {
    if (nblocks <= 0) return hipSuccess;
    TG_LAUNCH(k_quantize_q8k, dim3(lg_cdiv(nblocks, 4)), dim3(256), 0, st, x, static_cast<Q8K *>(xq), nblocks);
    return hipGetLastError();
}

hipError_t launch_matmul_q4k(const uint8_t *W, const void *xq, float *y, int nrows, int bpr, hipStream_t st) {
    if (nrows <= 0) return hipSuccess;
    // fewer rows per wave where that keeps about 1024 waves in the launch
    int R = q4k_rows_per_wave(bpr);
    while (R > 1 && nrows / R < 1024) R /= 2;
    TG_LAUNCH(k_matmul_q4k, dim3(lg_cdiv(nrows, 4 * R)), dim3(256), 0, st, W, static_cast<const Q8K *>(xq), y, nrows,
              bpr, R);
    return hipGetLastError();
}

hipError_t launch_matmul_q6k(const uint8_t *W, const void *xq, float *y, int nrows, int bpr, hipStream_t st) {
    if (nrows <= 0) return hipSuccess;
    int R = q4k_rows_per_wave(bpr);  // the same rows per wave as Q4_K
    while (R > 1 && nrows / R < 1024) R /= 2;
    TG_LAUNCH(k_matmul_q6k, dim3(lg_cdiv(nrows, 4 * R)), dim3(256), 0, st, W, static_cast<const Q8K *>(xq), y, nrows,
              bpr, R);
    return hipGetLastError();
}

hipError_t launch_matvec_two_acc(const void *A, bool half, const float *x, float *y, int nrows, int ncols,
                                 hipStream_t st) {
    if (nrows <= 0) return hipSuccess;
    const dim3 grid(lg_cdiv(nrows, 32));
    if (half)
        TG_LAUNCH(k_matvec_two_acc<true>, grid, dim3(256), 0, st, A, x, y, nrows, ncols);
    else
        TG_LAUNCH(k_matvec_two_acc<false>, grid, dim3(256), 0, st, A, x, y, nrows, ncols);
    return hipGetLastError();
}

hipError_t launch_rms_norm(const float *x, const float *w, float *out, int dim, float eps, hipStream_t st) {
    return launch_rms_norm_rows(x, w, out, dim, 1, eps, st);
}

hipError_t launch_rms_norm_rows(const float *x, const float *w, float *out, int dim, int rows, float eps,
                                hipStream_t st) {
    if (dim <= 0 || rows <= 0) return hipSuccess;
    TG_LAUNCH(k_rms_norm, dim3(rows), dim3(256), 0, st, x, w, out, dim, eps);
    return hipGetLastError();
}

hipError_t launch_matmul_q4k_scalar(const uint8_t *W, const float *x, float *y, int nrows, int bpr, hipStream_t st) {
    if (nrows <= 0) return hipSuccess;
    TG_LAUNCH(k_matmul_q4k_scalar, dim3(lg_cdiv(nrows, 256)), dim3(256), 0, st, W, x, y, nrows, bpr);
    return hipGetLastError();
}

hipError_t launch_silu_mul_vec(const float *g, const float *u, float *h, int n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    TG_LAUNCH(k_silu_mul_vec, dim3(lg_cdiv(n, 256)), dim3(256), 0, st, g, u, h, n);
    return hipGetLastError();
}

hipError_t launch_rope(float *x, int n_heads, int hd, const float *c, const float *sn, hipStream_t st) {
    const int n = n_heads * (hd / 2);
    if (n <= 0) return hipSuccess;
    TG_LAUNCH(k_rope, dim3(lg_cdiv(n, 256)), dim3(256), 0, st, x, n_heads, hd, c, sn);
    return hipGetLastError();
}

hipError_t launch_kv_append(const float *kn, const float *v, float *kc, float *vc, int n_kv, int seq, int hd, int row,
                            hipStream_t st) {
    if (n_kv * hd <= 0) return hipSuccess;
    TG_LAUNCH(k_kv_append, dim3(lg_cdiv((long)n_kv * hd, 256)), dim3(256), 0, st, kn, v, kc, vc, n_kv, seq, hd, row);
    return hipGetLastError();
}

static int att_ngrp(int ratio) { return (ratio + ATT_HB - 1) / ATT_HB; }

hipError_t launch_attn_scores(const float *q, const float *kc, float *scr, int n_heads, int seq, int hd, int ratio,
                              float inv_sqrt, hipStream_t st) {
    if (hd > 512 || hd < 2 || n_heads <= 0 || seq <= 0 || ratio <= 0 || n_heads % ratio) return hipErrorInvalidValue;
    const int ngrp = att_ngrp(ratio), n_kv = n_heads / ratio;
    const size_t lds = sizeof(float) * ((size_t)ATT_HB * hd + (size_t)ATT_TP * (hd + 1));
    const dim3 grid(attn_score_blocks(seq), n_kv * ngrp);
    if (hd % 4 == 0)
        TG_LAUNCH(k_attn_scores<true>, grid, dim3(256), lds, st, q, kc, scr, n_heads, seq, hd, ratio, ngrp, inv_sqrt);
    else
        TG_LAUNCH(k_attn_scores<false>, grid, dim3(256), lds, st, q, kc, scr, n_heads, seq, hd, ratio, ngrp, inv_sqrt);
    return hipGetLastError();
}

hipError_t launch_attn_softmax(float *scr, int n_heads, int seq, hipStream_t st) {
    if (n_heads <= 0 || seq <= 0) return hipErrorInvalidValue;
    TG_LAUNCH(k_attn_softmax, dim3(n_heads), dim3(256), 0, st, scr, n_heads, seq, attn_score_blocks(seq),
              attn_w_offset(n_heads, seq));
    return hipGetLastError();
}

hipError_t launch_attn_wv(const float *scr, const float *vc, float *out, int n_heads, int seq, int hd, int ratio,
                          hipStream_t st) {
    if (hd > 512 || hd < 2 || n_heads <= 0 || seq <= 0 || ratio <= 0 || n_heads % ratio) return hipErrorInvalidValue;
    const int ngrp = att_ngrp(ratio), n_kv = n_heads / ratio;
    const dim3 grid(lg_cdiv(hd, ATT_DS), n_kv * ngrp);
    const size_t woff = attn_w_offset(n_heads, seq);
    if (hd % 4 == 0)
        TG_LAUNCH(k_attn_wv<true>, grid, dim3(128), 0, st, scr, vc, out, seq, hd, ratio, ngrp, woff);
    else
        TG_LAUNCH(k_attn_wv<false>, grid, dim3(128), 0, st, scr, vc, out, seq, hd, ratio, ngrp, woff);
    return hipGetLastError();
}

hipError_t launch_argmax(const float *x, int n, float *pv, int *pi, int *out, hipStream_t st) {
    if (n <= 0) return hipErrorInvalidValue;
    const int nb = (int)std::min<long>(ARGMAX_BLOCKS, (long)lg_cdiv(n, 256));
    TG_LAUNCH(k_argmax_part, dim3(nb), dim3(256), 0, st, x, n, pv, pi);
    TG_LAUNCH(k_argmax_final, dim3(1), dim3(256), 0, st, pv, pi, nb, out);
    return hipGetLastError();
}

hipError_t launch_add_vec(float *x, const float *a, int n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    TG_LAUNCH(k_add_vec, dim3(lg_cdiv(n, 256)), dim3(256), 0, st, x, a, n);
    return hipGetLastError();
}

// the fused launches' shapes (x's Q8 blocks in at most 34.8 KB of LDS)
bool moe_q4k_ok(int n_exp, int embed, int inter) {
    return n_exp > 0 && n_exp <= LG_MOE_MAX && embed > 0 && inter > 0 && embed % LG_QK == 0 &&
           inter % LG_QK == 0 && embed / LG_QK <= 128;
}

hipError_t launch_moe_gateup_q4k(const LgMoeOps &P, int n_exp, const float *x, float *gu, int embed, int inter,
                                 hipStream_t st) {
    if (!moe_q4k_ok(n_exp, embed, inter)) return hipErrorInvalidValue;
    const int bpr = embed / LG_QK;
    TG_LAUNCH(k_moe_gateup_q4k, dim3(lg_cdiv(n_exp * 2 * inter, 4 * q4k_rows_per_wave(bpr))), dim3(256),
              8 + (size_t)bpr * LG_XQ_LDS, st, P, x, gu, n_exp, inter, bpr);
    return hipGetLastError();
}

hipError_t launch_moe_silu_q8k(const float *gu, void *hq, int n_exp, int inter, hipStream_t st) {
    if (!moe_q4k_ok(n_exp, LG_QK, inter)) return hipErrorInvalidValue;
    TG_LAUNCH(k_moe_silu_q8k, dim3(lg_cdiv(n_exp * (inter / LG_QK), 4)), dim3(256), 0, st, gu,
              static_cast<Q8K *>(hq), n_exp, inter);
    return hipGetLastError();
}

hipError_t launch_moe_down_acc_q4k(const LgMoeOps &P, int n_exp, const void *hq, float *out, int embed, int inter,
                                   bool add_to_out, hipStream_t st) {
    if (!moe_q4k_ok(n_exp, embed, inter)) return hipErrorInvalidValue;
    TG_LAUNCH(k_moe_down_acc_q4k, dim3(lg_cdiv(embed, 4)), dim3(256), 0, st, P, static_cast<const Q8K *>(hq), out,
              n_exp, embed, inter / LG_QK, add_to_out ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_acc_scaled(float *out, const float *v, float w, int n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    TG_LAUNCH(k_acc_scaled, dim3(lg_cdiv(n, 256)), dim3(256), 0, st, out, v, w, n);
    return hipGetLastError();
}

}  // namespace tg
