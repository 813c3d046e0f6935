// tg_persist.hip -- one-token decode of a whole MoE stack in one launch.
//
// The per-layer three-kernel path pays a kernel boundary (drain, launch,
// first-load latency) three times per layer.  Here one cooperative launch
// of one block per CU runs every layer of the stack; the blocks hand data to
// each other through tagged words instead of kernel boundaries.
//
// Units of one layer:
//   gate/up unit (j, m)  rows [32m, 32m+32) of gate and up of the j-th
//                        selected expert -> h rows -> Q8_0 block m of h_j
//   down unit g          rows [32g, 32g+32) of down for all k experts,
//                        combine, residual -> x rows (kept in LDS by the
//                        unit's block for the whole launch); the next
//                        layer's router and sum-of-squares partials of group g
//
// Hand-offs (each a tagged word array, see below):
//   down unit g -> down units   router + sum-of-squares partials of group g
//   down unit g -> gate/up      Q8_0 block g of x * s (s = the layer's RMS
//                               scale), and from unit 0 the k expert ids
//   gate/up (j, m) -> down      Q8_0 block m of h_j
// Every down unit derives the layer's routing itself from all partials
// (sum over groups in ascending order, top-k, softmax), so the routing is
// one hand-off away from the previous layer's down units.
//
// Tagged words.  A 64-bit word holds a 32-bit payload and a 32-bit tag
// (launch generation << 8 | layer + 1) and is stored and loaded with relaxed
// agent-scope atomics, so a reader that sees the expected tag sees the
// payload stored with it; no fence and no counter is needed, and every
// array is written once per layer.  Cross-layer reuse is safe by the data
// dependencies (a slot is rewritten only after every reader of its previous
// value has published something the writer had to read first); the router
// partials are double-buffered because a down unit may publish layer l+1's
// partials while a slower one still reads layer l's.
//
// Every poll is bounded: a thread that runs out of tries sets the error and
// abort words and its block leaves; polls also stop when they see the abort
// word, so the grid always drains.
//
// Arithmetic is the per-layer kernels' (tg_moe.hip): the same block-sum
// formula, the same sequential fma chains over blocks, the same grouped sums
// of squares and router dots, the same top-k keys and softmax, the same
// combine order, so results are bit-identical to that path and to the host
// definition.
#include "tg_device.h"
#include "tg_internal.h"

namespace tg {

constexpr int PS_GROUP = 32;                 // rows per unit = one Q8_0 block / one router group
constexpr int PS_QW = 10;                    // words of one published Q8_0 block: 8 x 4 bytes, d, sum
constexpr uint32_t PS_SPIN_LIMIT = 1u << 20; // tries of one poll
constexpr int PS_KT = 8;                     // top-k held in registers by a down unit

// status words: [0] abort, [1] error (1 = a poll ran out of tries)
enum { SY_ABORT = 0, SY_ERR = 1 };

__global__ void k_persist_reset(uint32_t *sync) {
    if (threadIdx.x < 4) sync[threadIdx.x] = 0u;
}

struct PersistArgs {
    const uint8_t *experts;  // arena experts, layer stride s.LB (tensor-planar)
    const float *routers;    // arena routers, layer stride E * H
    Shape s;
    int layer0, nl;
    float eps;
    float *x;                // [H] in / out
    uint64_t *rpw;           // [2][U_d][E + 1] router partials, sum of squares last
    uint64_t *xqw;           // [nbH][PS_QW]  Q8_0 blocks of x * s
    uint64_t *idw;           // [k]           expert ids
    uint64_t *hqw;           // [k][nbI][PS_QW] Q8_0 blocks of h
    uint32_t *sync;
    int32_t *idx_out;        // optional [nl][k]
    float *w_out;            // optional [nl][k]
    uint32_t gen;            // launch generation (1 .. 2^24 - 1)
    uint64_t *tl;            // optional timeline [nl][gridDim.x][PS_TL] wall-clock stamps
    int ug, ud, nunits;      // gate/up units (k * I/32), down units (H/32), total
    int log2_nbH;
};

TG_DEV uint32_t ps_tag(const PersistArgs &A, int l) { return (A.gen << 8) | (uint32_t)(l + 1); }

// Timeline stamps (wall clock) per block and layer, when A.tl is set:
//   0 layer start   1 routing known (down) / ids received (gate/up)
//   2 Q8_0 x published (down) / Q8_0 x received (gate/up)
//   3 h block published (gate/up)   4 down loads issued   5 h received
//   6 partials of the next layer published
constexpr int PS_TL = 8;

TG_DEV void ps_stamp(const PersistArgs &A, int l, int slot) {
    if (A.tl && threadIdx.x == 0) A.tl[((size_t)l * gridDim.x + blockIdx.x) * PS_TL + slot] = wall_clock64();
}

// ------------------------------------------------------------ tagged words

// Reads n tagged words into dst (LDS payloads).  Each thread owns the words
// i = tid + u * NT; per round it loads every word of a batch that is still
// missing (all loads in flight together), keeps the ones that carry `tag`,
// and sleeps briefly before the next round.  Rounds are bounded: a thread
// that runs out sets the error and abort words; every thread stops when it
// sees the abort word.  Block-wide; returns the same verdict in every thread.
template <int NT, int BATCH>
TG_DEV bool ll_read(const uint64_t *src, uint32_t *dst, int n, uint32_t tag, uint32_t *sync, int *flag) {
    static_assert(BATCH <= 64, "pending mask is 64 bits");
    const int tid = threadIdx.x;
    if (tid == 0) *flag = 1;
    __syncthreads();
    bool ok = true;
    for (int base = 0; base < n && ok; base += NT * BATCH) {
        uint64_t pend = 0;
#pragma unroll
        for (int u = 0; u < BATCH; u++)
            if (base + u * NT + tid < n) pend |= 1ull << u;
        uint32_t rounds = 0;
        while (pend) {
            uint64_t w[BATCH];
#pragma unroll
            for (int u = 0; u < BATCH; u++)
                if (pend >> u & 1ull) w[u] = ll_get(src + base + u * NT + tid);
#pragma unroll
            for (int u = 0; u < BATCH; u++) {
                if ((pend >> u & 1ull) && (uint32_t)(w[u] >> 32) == tag) {
                    dst[base + u * NT + tid] = (uint32_t)w[u];
                    pend &= ~(1ull << u);
                }
            }
            if (!pend) break;
            if (++rounds >= PS_SPIN_LIMIT) {
                __hip_atomic_store(sync + SY_ERR, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(sync + SY_ABORT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok = false;
                break;
            }
            if ((rounds & 63u) == 0u &&
                __hip_atomic_load(sync + SY_ABORT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) {
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    if (!ok) *flag = 0;
    __syncthreads();
    const bool res = *flag != 0;
    __syncthreads();
    return res;
}

// ------------------------------------------------------------------ LDS
struct PsLds {
    uint64_t *keys;   // [MAX_E]
    float *logit;     // [MAX_E]
    int *sidx;        // [MAX_K]
    float *sw;        // [MAX_K]
    float *sex;       // [MAX_K]
    float *misc;      // [4]: s, Q8_0 scale and sum being published
    int *flag;        // [4]
    float *xr;        // [32] this block's x rows (down unit)
    int *qtmp;        // [32] Q8_0 values being packed
    float *xd;        // [nbH r4]
    int *xs;          // [nbH r4]
    float *hd;        // [k * nbI r4]
    int *hs;          // [k * nbI r4]
    float *U;         // [max(64 * (nbH r4 + 4), k * 32 * (nbI r4 + 4))]
    float *D;         // [max(k, 2) * 32]
    float *wr;        // [E * 33] router slice of the next layer
    uint32_t *stage;  // tagged-word payloads: max(U_d * (E + 1), nbH * 10, k * nbI * 10)
};

__host__ __device__ inline int r4(int n) { return (n + 3) & ~3; }

__host__ __device__ inline size_t ps_u_floats(const Shape &s) {
    size_t a = (size_t)64 * (r4(s.nbH) + 4);
    size_t b = (size_t)s.k * PS_GROUP * (r4(s.nbI) + 4);
    return a > b ? a : b;
}

__host__ __device__ inline int ps_d_floats(const Shape &s) {
    return s.k * PS_GROUP > 2 * PS_GROUP ? s.k * PS_GROUP : 2 * PS_GROUP;
}

__host__ __device__ inline size_t ps_stage_words(const Shape &s, int ud) {
    size_t a = (size_t)ud * (s.E + 1);
    size_t b = (size_t)s.nbH * PS_QW;
    size_t c = (size_t)s.k * s.nbI * PS_QW;
    size_t m = a > b ? a : b;
    return m > c ? m : c;
}

__host__ __device__ inline size_t ps_lds_bytes(const Shape &s, int ud) {
    size_t b = 0;
    b += 8 * (size_t)MAX_E + 4 * (size_t)MAX_E;  // keys logit
    b += 4 * 3 * (size_t)MAX_K + 16 + 16;        // sidx sw sex misc flag
    b += 4 * 32 + 4 * 32;                        // xr qtmp
    b += 4 * (size_t)r4(s.nbH) * 2;              // xd xs
    b += 4 * (size_t)s.k * r4(s.nbI) * 2;        // hd hs
    b += 4 * ps_u_floats(s);                     // U
    b += 4 * (size_t)ps_d_floats(s);             // D
    b += 4 * (size_t)s.E * 33;                   // wr
    b += 4 * ps_stage_words(s, ud);              // stage
    return b;
}

TG_DEV PsLds ps_lds(uint8_t *base, const Shape &s, int ud) {
    PsLds L;
    uint8_t *p = base;
    L.keys = reinterpret_cast<uint64_t *>(p); p += 8 * MAX_E;
    L.logit = reinterpret_cast<float *>(p); p += 4 * MAX_E;
    L.sidx = reinterpret_cast<int *>(p); p += 4 * MAX_K;
    L.sw = reinterpret_cast<float *>(p); p += 4 * MAX_K;
    L.sex = reinterpret_cast<float *>(p); p += 4 * MAX_K;
    L.misc = reinterpret_cast<float *>(p); p += 16;
    L.flag = reinterpret_cast<int *>(p); p += 16;
    L.xr = reinterpret_cast<float *>(p); p += 4 * 32;
    L.qtmp = reinterpret_cast<int *>(p); p += 4 * 32;
    L.xd = reinterpret_cast<float *>(p); p += 4 * r4(s.nbH);
    L.xs = reinterpret_cast<int *>(p); p += 4 * r4(s.nbH);
    L.hd = reinterpret_cast<float *>(p); p += 4 * s.k * r4(s.nbI);
    L.hs = reinterpret_cast<int *>(p); p += 4 * s.k * r4(s.nbI);
    L.U = reinterpret_cast<float *>(p); p += 4 * ps_u_floats(s);
    L.D = reinterpret_cast<float *>(p); p += 4 * ps_d_floats(s);
    L.wr = reinterpret_cast<float *>(p); p += 4 * s.E * 33;
    L.stage = reinterpret_cast<uint32_t *>(p);
    (void)ud;
    return L;
}

// NaN ranks as -inf, -0 as +0; (logit desc, index asc) as one 64-bit key.
TG_DEV uint64_t ps_rank_key(float l, int e) {
    float v = l != l ? -__builtin_inff() : l;
    v = v + 0.0f;
    uint32_t u = __float_as_uint(v);
    uint32_t mono = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)mono << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)e);
}

// ------------------------------------------------------------ routing
// Routing of layer l from all groups' partials (down units): s, logits,
// top-k ids (LDS sidx, descending logit, ties to the lower index), softmax
// weights (LDS sw).  False if a poll gave up.
template <int NT>
TG_DEV bool ps_route(const PersistArgs &A, int l, PsLds &L) {
    const Shape &s = A.s;
    const int tid = threadIdx.x, E = s.E, ud = A.ud, row = E + 1;
    if (!ll_read<NT, 36>(A.rpw + (size_t)(l & 1) * ud * row, L.stage, ud * row, ps_tag(A, l), A.sync, L.flag))
        return false;
    const float *P = reinterpret_cast<const float *>(L.stage);
    if (tid == NT - 1) {
        // sum of squares: group partials added in ascending order
        float tot = 0.0f;
        for (int g = 0; g < ud; g++) tot = tot + P[g * row + E];
        L.misc[0] = rms_scale(tot, s.H, A.eps);
    }
    if (tid < s.k) L.sidx[tid] = 0;
    float raw = 0.0f;
    if (tid < E)
        for (int g = 0; g < ud; g++) raw = raw + P[g * row + tid];
    __syncthreads();
    if (tid < E) {
        const float lg = raw * L.misc[0];
        L.logit[tid] = lg;
        L.keys[tid] = ps_rank_key(lg, tid);
    }
    __syncthreads();
    // rank = number of larger keys (tpe threads per expert)
    {
        const int tpe = E * 4 <= NT ? 4 : (E * 2 <= NT ? 2 : 1);
        const int e = tid / tpe, part = tid - e * tpe;
        int cnt = 0;
        if (e < E) {
            const uint64_t my = L.keys[e];
            const int n = E / tpe, b0 = part * n;
            for (int i = 0; i < n; i++) cnt += L.keys[b0 + i] > my ? 1 : 0;
        }
        if (tpe >= 2) cnt += __shfl_xor(cnt, 1, WAVE);
        if (tpe >= 4) cnt += __shfl_xor(cnt, 2, WAVE);
        if (e < E && part == 0 && cnt < s.k) L.sidx[cnt] = e;
    }
    __syncthreads();
    if (tid == 0) {
        const int k = s.k;
        const float lmax = L.logit[L.sidx[0]];
        for (int i = 0; i < k; i++) L.sex[i] = expf_tg(L.logit[L.sidx[k - 1 - i]] - lmax);
        const float sum = np_pairwise_sum(L.sex, k);
        for (int i = 0; i < k; i++) L.sw[k - 1 - i] = L.sex[i] / sum;
    }
    __syncthreads();
    return true;
}

// Q8_0 of one 32-value block held by lanes 0..31 of wave 0 (v = this lane's
// value), published as PS_QW tagged words: 8 words of 4 packed values, then
// float(half d), then the block sum.  Must be called by the whole block.
TG_DEV void ps_publish_q8(float v, uint64_t *dst, uint32_t tag, PsLds &L) {
    const int tid = threadIdx.x;
    if (tid < 32) {
        float dq; int qsum; uint16_t dh;
        const int q = q8_lane(v, dq, qsum, dh);
        L.qtmp[tid] = q;
        if (tid == 0) {
            L.misc[1] = dq;
            reinterpret_cast<int *>(L.misc)[2] = qsum;
        }
    }
    __syncthreads();
    if (tid < PS_QW) {
        uint32_t word;
        if (tid < 8) {
            word = (uint32_t)(L.qtmp[4 * tid] & 255) | ((uint32_t)(L.qtmp[4 * tid + 1] & 255) << 8) |
                   ((uint32_t)(L.qtmp[4 * tid + 2] & 255) << 16) | ((uint32_t)(L.qtmp[4 * tid + 3] & 255) << 24);
        } else if (tid == 8) {
            word = __float_as_uint(L.misc[1]);
        } else {
            word = (uint32_t)reinterpret_cast<const int *>(L.misc)[2];
        }
        ll_put(dst + tid, word, tag);
    }
    __syncthreads();
}

TG_DEV float ps_chain4(const float *U, const float *dx, int nb) {
    float acc = 0.0f;
    const float4 *u4 = reinterpret_cast<const float4 *>(U);
    const float4 *d4 = reinterpret_cast<const float4 *>(dx);
    int q = 0;
    for (; q < nb / 4; q++) {
        float4 u = u4[q], d = d4[q];
        acc = __builtin_fmaf(u.x, d.x, acc);
        acc = __builtin_fmaf(u.y, d.y, acc);
        acc = __builtin_fmaf(u.z, d.z, acc);
        acc = __builtin_fmaf(u.w, d.w, acc);
    }
    for (int b = 4 * q; b < nb; b++) acc = __builtin_fmaf(U[b], dx[b], acc);
    return acc;
}

// ------------------------------------------------------------ router slice
// Router slice [E][32] of layer `layer`, columns [32g, 32g+32): float4
// chunk c of the E * 8 chunks goes to thread c % NT, slot c / NT.
constexpr int PS_WR_SLOTS = 4;  // E * 8 <= NT * PS_WR_SLOTS

template <int NT>
TG_DEV void ps_wr_load(const PersistArgs &A, int layer, int g, float4 (&wv)[PS_WR_SLOTS]) {
    const int tid = threadIdx.x, E = A.s.E, H = A.s.H;
#pragma unroll
    for (int v = 0; v < PS_WR_SLOTS; v++) {
        const int c = v * NT + tid;
        wv[v] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (c < E * 8) {
            const int e = c >> 3, o = (c & 7) * 4;
            wv[v] = *reinterpret_cast<const float4 *>(A.routers + (size_t)layer * E * H + (size_t)e * H +
                                                      g * PS_GROUP + o);
        }
    }
}

template <int NT>
TG_DEV void ps_wr_store(const PersistArgs &A, const float4 (&wv)[PS_WR_SLOTS], PsLds &L) {
    const int tid = threadIdx.x, E = A.s.E;
#pragma unroll
    for (int v = 0; v < PS_WR_SLOTS; v++) {
        const int c = v * NT + tid;
        if (c < E * 8) {
            const int e = c >> 3, o = (c & 7) * 4;
            float *w = L.wr + e * 33 + o;
            w[0] = wv[v].x; w[1] = wv[v].y; w[2] = wv[v].z; w[3] = wv[v].w;
        }
    }
}

// Group g's partials of layer l (router dots: fma chain over the group's 32
// rows, one thread per expert; sum of squares) from the LDS router slice and
// x rows, published to slot l & 1.
template <int NT>
TG_DEV void ps_publish_partials(const PersistArgs &A, int l, int g, PsLds &L) {
    const int tid = threadIdx.x, E = A.s.E;
    uint64_t *dst = A.rpw + ((size_t)(l & 1) * A.ud + g) * (E + 1);
    const uint32_t tag = ps_tag(A, l);
    if (tid < E) {
        float a = 0.0f;
        const float *w = L.wr + tid * 33;
        for (int i = 0; i < PS_GROUP; i++) a = __builtin_fmaf(w[i], L.xr[i], a);
        ll_put(dst + tid, __float_as_uint(a), tag);
    }
    if (tid == NT - 1) {
        float a = 0.0f;
        for (int i = 0; i < PS_GROUP; i++) a = __builtin_fmaf(L.xr[i], L.xr[i], a);
        ll_put(dst + E, __float_as_uint(a), tag);
    }
}

// ------------------------------------------------------------ gate / up
// Gate/up unit u = (j, m) of layer l.  Item mapping: nbH is a power of two
// dividing NT, so thread t always owns block column b = t % nbH; its v-th
// item is row-dot rd = v * (NT / nbH) + t / nbH (gate rows 0..31, then up
// rows 32..63).  `first`: this block's first unit of the layer, which reads
// the expert ids and Q8_0(x * s).
template <int NT, int GUI>
TG_DEV bool ps_gateup_unit(const PersistArgs &A, const uint8_t *lp, int l, int u, bool first, PsLds &L) {
    const Shape &s = A.s;
    const int tid = threadIdx.x, nbH = s.nbH, nbI = s.nbI, I = s.I;
    const uint32_t tag = ps_tag(A, l);
    if (first && !ll_read<NT, 1>(A.idw, reinterpret_cast<uint32_t *>(L.sidx), s.k, tag, A.sync, L.flag))
        return false;
    if (first) ps_stamp(A, l, 1);
    const int j = (int)fdiv((uint32_t)u, s.divI), m = u - j * nbI;
    const uint8_t *ex = lp + (size_t)L.sidx[j] * s.EB;
    const size_t ntb = (size_t)I * nbH;
    const int b = tid & (nbH - 1);
    const int r0 = tid >> A.log2_nbH;
    const int rstep = NT >> A.log2_nbH;
    const size_t o0 = (size_t)m * PS_GROUP * nbH + b;
    uint4 gw[GUI];
    uint16_t gd[GUI];
#pragma unroll
    for (int v = 0; v < GUI; v++) {
        const int rd = v * rstep + r0;
        gw[v] = make_uint4(0u, 0u, 0u, 0u);
        gd[v] = 0;
        if (rd < 2 * PS_GROUP) {
            const int mat = rd >> 5;
            const uint8_t *tb = ex + (size_t)mat * s.GB;
            const size_t o = o0 + (size_t)(rd & 31) * nbH;
            gw[v] = reinterpret_cast<const uint4 *>(tb)[o];
            gd[v] = reinterpret_cast<const uint16_t *>(tb + ntb * 16)[o];
        }
    }
    if (first) {
        // Q8_0(x * s) while the loads are in flight
        if (!ll_read<NT, 4>(A.xqw, L.stage, nbH * PS_QW, tag, A.sync, L.flag)) return false;
        ps_stamp(A, l, 2);
        for (int i = tid; i < nbH; i += NT) {
            L.xd[i] = __uint_as_float(L.stage[i * PS_QW + 8]);
            L.xs[i] = (int)L.stage[i * PS_QW + 9];
        }
        __syncthreads();
    }
    const int ust = r4(nbH) + 4;
    const int xsb = L.xs[b];
    const int *xqb = reinterpret_cast<const int *>(L.stage + b * PS_QW);
#pragma unroll
    for (int v = 0; v < GUI; v++) {
        const int rd = v * rstep + r0;
        if (rd < 2 * PS_GROUP) {
            const int S = dot_q4_q8(gw[v], xqb) - 8 * xsb;
            L.U[rd * ust + b] = (float)S * h2f(gd[v]);
        }
    }
    __syncthreads();
    if (tid < 64) L.D[tid] = ps_chain4(L.U + tid * ust, L.xd, nbH);
    __syncthreads();
    const float hv = tid < 32 ? silu_mul(L.D[tid], L.D[32 + tid]) : 0.0f;
    ps_publish_q8(hv, A.hqw + ((size_t)j * nbI + m) * PS_QW, tag, L);
    ps_stamp(A, l, 3);
    return true;
}

// ------------------------------------------------------------ down
// Down unit g of layer l: loads first (they stream while the gate/up units
// run), then Q8_0 h of the k experts, dots, chains, combine, x rows, and
// the next layer's partials of group g.  Item mapping: thread t owns the
// (row, block) slots q = v * NT + t (v < QV) of the unit's 32 x nbI grid and
// loads that slot of each of the k experts.
template <int NT, int QV>
TG_DEV bool ps_down_unit(const PersistArgs &A, const uint8_t *lp, int l, int g, PsLds &L) {
    const Shape &s = A.s;
    const int tid = threadIdx.x, nbI = s.nbI, H = s.H, k = s.k;
    const int per = PS_GROUP * nbI;  // slots of one expert
    const size_t ntb = (size_t)H * nbI;
    const size_t o0 = (size_t)g * per;
    const bool more = l + 1 < A.nl;
    uint4 dw[PS_KT][QV];
    uint16_t dd[PS_KT][QV];
#pragma unroll
    for (int j = 0; j < PS_KT; j++) {
        const uint8_t *tb = lp + (size_t)L.sidx[j < k ? j : 0] * s.EB + 2 * s.GB;
#pragma unroll
        for (int v = 0; v < QV; v++) {
            const int q = v * NT + tid;
            dw[j][v] = make_uint4(0u, 0u, 0u, 0u);
            dd[j][v] = 0;
            if (j < k && q < per) {
                dw[j][v] = reinterpret_cast<const uint4 *>(tb)[o0 + q];
                dd[j][v] = reinterpret_cast<const uint16_t *>(tb + ntb * 16)[o0 + q];
            }
        }
    }
    float4 wrv[PS_WR_SLOTS];
    if (more) ps_wr_load<NT>(A, A.layer0 + l + 1, g, wrv);
    ps_stamp(A, l, 4);

    if (!ll_read<NT, 8>(A.hqw, L.stage, k * nbI * PS_QW, ps_tag(A, l), A.sync, L.flag)) return false;
    ps_stamp(A, l, 5);
    const int nbp = r4(nbI);
    for (int i = tid; i < k * nbI; i += NT) {
        const int j = (int)fdiv((uint32_t)i, s.divI), b = i - j * nbI;
        L.hd[j * nbp + b] = __uint_as_float(L.stage[i * PS_QW + 8]);
        L.hs[j * nbp + b] = (int)L.stage[i * PS_QW + 9];
    }
    if (more) ps_wr_store<NT>(A, wrv, L);
    __syncthreads();
    const int ust = nbp + 4;
#pragma unroll
    for (int v = 0; v < QV; v++) {
        const int q = v * NT + tid;
        if (q < per) {
            const int row = (int)fdiv((uint32_t)q, s.divI), b = q - row * nbI;
#pragma unroll
            for (int j = 0; j < PS_KT; j++) {
                if (j < k) {
                    const int *hqb = reinterpret_cast<const int *>(L.stage + ((size_t)j * nbI + b) * PS_QW);
                    const int S = dot_q4_q8(dw[j][v], hqb) - 8 * L.hs[j * nbp + b];
                    L.U[(j * PS_GROUP + row) * ust + b] = (float)S * h2f(dd[j][v]);
                }
            }
        }
    }
    __syncthreads();
    for (int rd = tid; rd < k * PS_GROUP; rd += NT)
        L.D[rd] = ps_chain4(L.U + rd * ust, L.hd + (rd >> 5) * nbp, nbI);
    __syncthreads();
    if (tid < PS_GROUP) {
        float acc = 0.0f;
        for (int jj = k - 1; jj >= 0; jj--) acc = __builtin_fmaf(L.sw[jj], L.D[jj * PS_GROUP + tid], acc);
        L.xr[tid] = L.xr[tid] + acc;
    }
    __syncthreads();
    if (more) ps_publish_partials<NT>(A, l + 1, g, L);
    ps_stamp(A, l, 6);
    return true;
}

// ------------------------------------------------------------ kernel
template <int NT, int GUI, int QV>
__global__ __launch_bounds__(NT) void k_persist(PersistArgs A) {
    extern __shared__ __align__(16) uint8_t smem[];
    PsLds L = ps_lds(smem, A.s, A.ud);
    const int tid = threadIdx.x, G = gridDim.x, bid = blockIdx.x;
    const int k = A.s.k;

    // this block's units: bid, bid + G, ... (gate/up units first, then down);
    // the launcher guarantees at most two gate/up units and one down unit
    const int gu0 = bid < A.ug ? bid : -1;
    const int gu1 = bid + G < A.ug ? bid + G : -1;
    int dn = -1;
    for (int u = bid; u < A.nunits; u += G)
        if (u >= A.ug) dn = u - A.ug;

    // prologue: this block's x rows and layer 0's partials of its group
    if (dn >= 0) {
        float4 wv[PS_WR_SLOTS];
        ps_wr_load<NT>(A, A.layer0, dn, wv);
        if (tid < PS_GROUP) L.xr[tid] = A.x[dn * PS_GROUP + tid];
        ps_wr_store<NT>(A, wv, L);
        __syncthreads();
        ps_publish_partials<NT>(A, 0, dn, L);
    }

    for (int l = 0; l < A.nl; l++) {
        const uint8_t *lp = A.experts + (size_t)(A.layer0 + l) * A.s.LB;
        ps_stamp(A, l, 0);
        if (dn >= 0) {
            if (!ps_route<NT>(A, l, L)) return;
            ps_stamp(A, l, 1);
            const uint32_t tag = ps_tag(A, l);
            const float xs = tid < PS_GROUP ? L.xr[tid] * L.misc[0] : 0.0f;
            ps_publish_q8(xs, A.xqw + (size_t)dn * PS_QW, tag, L);
            ps_stamp(A, l, 2);
            if (dn == 0 && tid < k) {
                ll_put(A.idw + tid, (uint32_t)L.sidx[tid], tag);
                if (A.idx_out) A.idx_out[(size_t)l * k + tid] = L.sidx[tid];
                if (A.w_out) A.w_out[(size_t)l * k + tid] = L.sw[tid];
            }
        }
        if (gu0 >= 0 && !ps_gateup_unit<NT, GUI>(A, lp, l, gu0, true, L)) return;
        if (gu1 >= 0 && !ps_gateup_unit<NT, GUI>(A, lp, l, gu1, false, L)) return;
        if (dn >= 0 && !ps_down_unit<NT, QV>(A, lp, l, dn, L)) return;
    }
    if (dn >= 0 && tid < PS_GROUP) A.x[dn * PS_GROUP + tid] = L.xr[tid];
}

// ================================================================ launcher
struct PsVariant {
    int nt, gui, qv;
    const void *fn;
};

template <int NT, int GUI, int QV>
static const void *ps_fn() {
    return reinterpret_cast<const void *>(&k_persist<NT, GUI, QV>);
}

// smallest first; 256 threads = one wave per SIMD, so a wave may hold a
// whole unit's loads in registers
static const PsVariant kPsVariants[] = {
    {256, 2, 1, ps_fn<256, 2, 1>()},   {256, 4, 1, ps_fn<256, 4, 1>()},  {256, 8, 2, ps_fn<256, 8, 2>()},
    {256, 16, 3, ps_fn<256, 16, 3>()},
};

static const PsVariant *ps_pick(const Shape &s) {
    const int nbH = s.nbH;
    if (nbH & (nbH - 1)) return nullptr;  // power of two
    for (const auto &v : kPsVariants) {
        if (nbH > v.nt || 64 * nbH > v.gui * v.nt) continue;
        if (PS_GROUP * s.nbI > v.qv * v.nt) continue;
        if (s.E * 8 > v.nt * PS_WR_SLOTS || s.E > v.nt) continue;
        return &v;
    }
    return nullptr;
}

bool persist_shape_ok(const Shape &s) {
    return ps_pick(s) != nullptr && s.H % PS_GROUP == 0 && s.I % PS_GROUP == 0 && s.E <= MAX_E && s.E % 4 == 0 &&
           s.k <= PS_KT && ps_lds_bytes(s, s.H / PS_GROUP) <= 160 * 1024;
}

size_t persist_timeline_words(int nl, int n_cu) { return (size_t)nl * n_cu * PS_TL; }

size_t persist_scratch_bytes(const Shape &s) {
    size_t ud = (size_t)s.H / PS_GROUP;
    size_t words = 2 * ud * (s.E + 1) + (size_t)s.nbH * PS_QW + PS_KT + (size_t)s.k * s.nbI * PS_QW;
    return 8 * words;
}

hipError_t launch_persist(const uint8_t *experts, const float *routers, const Shape &s, int layer0, int nl, float eps,
                          float *x, void *scratch, uint32_t *sync, uint32_t gen, int32_t *idx_out, float *w_out,
                          uint64_t *timeline, size_t timeline_words, int n_cu, hipStream_t st) {
    const PsVariant *v = ps_pick(s);
    if (!v || !persist_shape_ok(s) || nl < 1 || nl > 254 || gen == 0 || gen >= (1u << 24))
        return hipErrorInvalidValue;
    PersistArgs A;
    A.experts = experts;
    A.routers = routers;
    A.s = s;
    A.layer0 = layer0;
    A.nl = nl;
    A.eps = eps;
    A.x = x;
    A.ud = s.H / PS_GROUP;
    A.ug = s.k * s.nbI;
    A.nunits = A.ug + A.ud;
    A.log2_nbH = 0;
    while ((1 << A.log2_nbH) < s.nbH) A.log2_nbH++;
    uint64_t *p = static_cast<uint64_t *>(scratch);
    A.rpw = p; p += 2 * (size_t)A.ud * (s.E + 1);
    A.xqw = p; p += (size_t)s.nbH * PS_QW;
    A.idw = p; p += PS_KT;
    A.hqw = p;
    A.sync = sync;
    A.idx_out = idx_out;
    A.w_out = w_out;
    A.gen = gen;
    A.tl = nullptr;

    size_t lds = ps_lds_bytes(s, A.ud);
    hipError_t e = hipFuncSetAttribute(v->fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    int per_cu = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, v->fn, v->nt, lds);
    if (e != hipSuccess) return e;
    if (per_cu < 1) return hipErrorInvalidConfiguration;
    // one block per CU: the units of a layer are spread over every CU
    const int G = n_cu < A.nunits ? n_cu : A.nunits;
    // a block holds at most two gate/up units and one down unit
    if ((A.ug + G - 1) / G > 2 || A.ud > G) return hipErrorInvalidConfiguration;
    if (timeline && timeline_words >= (size_t)nl * G * PS_TL) A.tl = timeline;
    TG_LAUNCH(k_persist_reset, dim3(1), dim3(64), 0, st, sync);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    void *args[] = {&A};
    return hipLaunchCooperativeKernel(v->fn, dim3(G), dim3(v->nt), args, (unsigned)lds, st);
}

}  // namespace tg
