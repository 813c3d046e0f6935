// tg_moe.hip -- the decode MoE block on gfx950: routing, gate/up + SwiGLU,
// down + weighted combine.
//
// Per layer three kernels, separated by kernel boundaries (replayed as a HIP
// graph, where a boundary costs little):
//
//   k_route_dec grid (E, T)        raw router dot of one expert for one token
//                                  and the token's RMS scale; the token's
//                                  last block ranks the logits (top-k,
//                                  softmax) and writes Q8_0(x * s)
//   k_gateup    grid (I/32, k, T)  32 rows of gate and up of one selected
//                                  expert, h = SiLU(gate) * up, Q8_0 block
//                                  of h
//   k_down      grid (H/RD, T)     RD rows of down for all k experts,
//                                  combine, residual
//
// Routing, the activation Q8_0 and the h Q8_0 happen once per token, so the
// weight-streaming kernels start their loads after one dependent read of
// the expert ids.  One CU streams only a few tens of GB/s from HBM, so every
// weight-streaming kernel spreads its bytes over at least one block per CU
// (256 CUs).
//
// Numerics: see tg_kernels.hip (row dots) and the routing definition below;
// every result is bit-identical to the host definition.
#include "tg_device.h"
#include "tg_internal.h"

namespace tg {

// ================================================================= routing
// Grouped sums: x is split in groups of RG = 32 consecutive elements.
//   raw[e] = sum over groups g (ascending) of the fma chain over the group
//            of W[e][i] * x[i]
//   ss     = the same grouping over x[i] * x[i]
//   s      = 1 / sqrt(ss / H + eps),  logit[e] = raw[e] * s
constexpr int RG = 32;
constexpr int RT_THREADS = 256;  // groups per k_route block (H <= 8192)

// Block (e, tb): expert e for tokens [8 tb, 8 tb + 8).  Thread (g, ts) runs
// the fma chain of group g for tokens ts, ts + TS, ... (TS = 256 / G token
// slots per pass), keeping the router group in registers; then one thread
// per token adds the G group sums in ascending order.
constexpr int RT_TOK = 8;

__global__ __launch_bounds__(RT_THREADS) void k_route(const float *__restrict__ Wr, const float *__restrict__ x, int T,
                                                      int E, int H, float *__restrict__ raw) {
    __shared__ __align__(16) float gp[RT_TOK][RT_THREADS];
    const int e = blockIdx.x, t0 = blockIdx.y * RT_TOK, tid = threadIdx.x, G = H / RG;
    const int TS = RT_THREADS / G, g = tid % G, ts = tid / G;
    if (ts < TS) {
        const float4 *w4 = reinterpret_cast<const float4 *>(Wr + (size_t)e * H + g * RG);
        float4 wv[RG / 4];
#pragma unroll
        for (int q = 0; q < RG / 4; q++) wv[q] = w4[q];
        for (int tt = ts; tt < RT_TOK; tt += TS) {
            const int t = t0 + tt;
            if (t >= T) break;
            const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)t * H + g * RG);
            float4 xv[RG / 4];
#pragma unroll
            for (int q = 0; q < RG / 4; q++) xv[q] = x4[q];
            float acc = 0.0f;
#pragma unroll
            for (int q = 0; q < RG / 4; q++) {
                acc = __builtin_fmaf(wv[q].x, xv[q].x, acc);
                acc = __builtin_fmaf(wv[q].y, xv[q].y, acc);
                acc = __builtin_fmaf(wv[q].z, xv[q].z, acc);
                acc = __builtin_fmaf(wv[q].w, xv[q].w, acc);
            }
            gp[tt][g] = acc;
        }
    }
    __syncthreads();
    if (tid < RT_TOK && t0 + tid < T) {
        const float4 *p4 = reinterpret_cast<const float4 *>(gp[tid]);
        float tot = 0.0f;
#pragma unroll 4
        for (int q = 0; q < G / 4; q++) {
            const float4 v = p4[q];
            tot = tot + v.x; tot = tot + v.y; tot = tot + v.z; tot = tot + v.w;
        }
        raw[(size_t)(t0 + tid) * E + e] = tot;
    }
}

// Few tokens (below 128): block = RS_T tokens x RS_E experts, 1024 threads.
// Thread (pair p = tid % RS_PAIRS, part j = tid / RS_PAIRS) runs the fma
// chains of pair p (token p / RS_E, expert p % RS_E) over the G / RS_PARTS
// consecutive groups of part j, two at a time; the chain sums meet in LDS and
// one thread per pair adds them in ascending group order, exactly as k_route
// does.  A block reads its RS_E router rows and RS_T token rows once (through
// the L1; every 64 lanes touch at most 2 rows of each).
constexpr int RS_T = 4, RS_E = 8, RS_PAIRS = RS_T * RS_E, RS_PARTS = 1024 / RS_PAIRS;

__host__ __device__ inline size_t route_small_lds(int H) { return 4 * (size_t)RS_PAIRS * (H / RG + 1); }

__global__ __launch_bounds__(1024) void k_route_small(const float *__restrict__ Wr, const float *__restrict__ x, int T,
                                                      int E, int H, float *__restrict__ raw) {
    extern __shared__ __align__(16) float cs[];  // [RS_PAIRS][G + 1]
    const int tid = threadIdx.x, p = tid % RS_PAIRS, j = tid / RS_PAIRS, G = H / RG, gp = G / RS_PARTS;
    const int t = blockIdx.x * RS_T + p / RS_E, e = blockIdx.y * RS_E + p % RS_E;
    if (t < T && e < E) {
        const float4 *w4 = reinterpret_cast<const float4 *>(Wr + (size_t)e * H);
        const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)t * H);
        for (int g = j * gp; g < (j + 1) * gp; g += 2) {  // gp is even
            float4 wa[RG / 4], xa[RG / 4], wb[RG / 4], xb[RG / 4];
#pragma unroll
            for (int q = 0; q < RG / 4; q++) {
                wa[q] = w4[g * (RG / 4) + q];
                xa[q] = x4[g * (RG / 4) + q];
                wb[q] = w4[(g + 1) * (RG / 4) + q];
                xb[q] = x4[(g + 1) * (RG / 4) + q];
            }
            float a = 0.0f, b = 0.0f;
#pragma unroll
            for (int q = 0; q < RG / 4; q++) {
                a = __builtin_fmaf(wa[q].x, xa[q].x, a);
                b = __builtin_fmaf(wb[q].x, xb[q].x, b);
                a = __builtin_fmaf(wa[q].y, xa[q].y, a);
                b = __builtin_fmaf(wb[q].y, xb[q].y, b);
                a = __builtin_fmaf(wa[q].z, xa[q].z, a);
                b = __builtin_fmaf(wb[q].z, xb[q].z, b);
                a = __builtin_fmaf(wa[q].w, xa[q].w, a);
                b = __builtin_fmaf(wb[q].w, xb[q].w, b);
            }
            cs[p * (G + 1) + g] = a;
            cs[p * (G + 1) + g + 1] = b;
        }
    }
    __syncthreads();
    if (tid < RS_PAIRS && t < T && e < E) {
        float tot = 0.0f;
        for (int g = 0; g < G; g++) tot = tot + cs[p * (G + 1) + g];
        raw[(size_t)t * E + e] = tot;
    }
}

// Few tokens, first half of the routing: block (g, tile) forms, for the
// RCT tokens of its tile and every expert, the fma chain of group g (its 32
// elements in order, from 0) and writes it to chains[g][t][e]; k_route_q8
// adds a token's chains in ascending group order, so the logits are k_route's
// bit for bit.  Every router and x element of a tile is read once (group g's
// columns staged in LDS).  Thread (ti, ej): tokens RCT/8 ti .. + RCT/8 - 1,
// experts ej + 32 b (b < 4; E <= 128), so a wave's router reads are 32
// consecutive rows (conflict-free at the 9-float4 row stride) and its stores
// coalesce.  Tiles of 16 tokens up to 64 tokens (256 blocks at H = 2048), of
// 32 above.
constexpr int RC_THREADS = 256;

__host__ __device__ inline bool route_chains_ok(int E, int H) { return E <= 128 && E % 32 == 0 && H % RG == 0; }

template <int RCT>
__global__ __launch_bounds__(RC_THREADS) void k_route_chains(const float *__restrict__ Wr, const float *__restrict__ x,
                                                             int T, int E, int H, float *__restrict__ chains) {
    constexpr int Q = RG / 4, QS = Q + 1;  // float4 per group row, padded stride
    constexpr int TPT = RCT / 8;           // tokens per thread
    static_assert(RCT % 8 == 0 && RC_THREADS == 8 * 32, "thread map");
    __shared__ float4 xs[RCT * QS];
    __shared__ float4 ws[128 * QS];
    const int g = blockIdx.x, t0 = blockIdx.y * RCT, tid = threadIdx.x;
    for (int i = tid; i < RCT * Q; i += RC_THREADS) {
        const int r = i / Q, q = i % Q, t = t0 + r;
        xs[r * QS + q] = t < T ? reinterpret_cast<const float4 *>(x + (size_t)t * H + (size_t)g * RG)[q]
                               : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int v = 0; v < 128 * Q / RC_THREADS; v++) {
        const int i = v * RC_THREADS + tid, e = i / Q, q = i % Q;
        if (e < E) ws[e * QS + q] = reinterpret_cast<const float4 *>(Wr + (size_t)e * H + (size_t)g * RG)[q];
    }
    __syncthreads();
    const int ti = tid >> 5, ej = tid & 31;
    float acc[TPT][4];
#pragma unroll
    for (int a = 0; a < TPT; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = 0.0f;
#pragma unroll
    for (int q = 0; q < Q; q++) {
        float4 xv[TPT], wv[4];
#pragma unroll
        for (int a = 0; a < TPT; a++) xv[a] = xs[(TPT * ti + a) * QS + q];
#pragma unroll
        for (int b = 0; b < 4; b++) wv[b] = ws[min(ej + 32 * b, E - 1) * QS + q];
#pragma unroll
        for (int a = 0; a < TPT; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                acc[a][b] = __builtin_fmaf(wv[b].x, xv[a].x, acc[a][b]);
                acc[a][b] = __builtin_fmaf(wv[b].y, xv[a].y, acc[a][b]);
                acc[a][b] = __builtin_fmaf(wv[b].z, xv[a].z, acc[a][b]);
                acc[a][b] = __builtin_fmaf(wv[b].w, xv[a].w, acc[a][b]);
            }
    }
#pragma unroll
    for (int a = 0; a < TPT; a++) {
        const int t = t0 + TPT * ti + a;
        if (t < T)
#pragma unroll
            for (int b = 0; b < 4; b++)
                if (ej + 32 * b < E) chains[((size_t)g * T + t) * E + ej + 32 * b] = acc[a][b];
    }
}

// Many tokens: block = 16 tokens x 32 experts, 256 threads (512 blocks at
// 2048 tokens, two resident per CU).  Four groups (128 consecutive elements)
// of x and of the router rows are staged in LDS per step, the next step's
// loads in flight while the current one is used.  Wave w runs the fma chains
// of group w of the step (with more groups per step, w + 4, ...) for all 512
// pairs: lane (ti, ej) takes tokens
// ti + 8 a (a < 2) and experts ej + 8 b (b < 4), 8 chains from 6 LDS values
// per element (consecutive rows per lane, conflict-free), element by element
// across the chains so consecutive fmas are independent.  The chains meet in
// LDS and thread p adds them to the totals of pairs p and p + 256 in
// ascending group order, exactly as k_route does.
constexpr int RTT_T = 16, RTT_E = 32;
constexpr int RT_CH = 4;                   // groups per staging step of the 4-wave form
constexpr int RT_PAIRS = RTT_T * RTT_E;    // 512

// NW waves per block, one group of each staging step per wave (NW = 8: 512
// threads, 8 groups of 32 elements staged per step, 66 KB of LDS; two blocks
// per CU keep four waves per SIMD where the 4-wave form kept two: 28.5 -> 25.0
// us at 2048 tokens)
template <int NW>
__global__ __launch_bounds__(NW * 64) void k_route_tiled(const float *__restrict__ Wr, const float *__restrict__ x,
                                                         int T, int E, int H, float *__restrict__ raw) {
    constexpr int NT = NW * 64, CH = NW;      // threads, groups per step
    constexpr int RW = CH * RG + 4;           // LDS row stride (floats)
    constexpr int F4 = CH * RG / 4;           // float4 per staged row and step
    __shared__ __align__(16) float xs[RTT_T][RW];
    __shared__ __align__(16) float ws[RTT_E][RW];
    __shared__ float cs[CH][RT_PAIRS];
    const int tid = threadIdx.x, t0 = blockIdx.x * RTT_T, e0 = blockIdx.y * RTT_E;
    const int gw = tid >> 6, ti = (tid >> 3) & 7, ej = tid & 7;
    // staging: thread loads rows r = tid / F4 + RS v, float4 column c4
    const int sr = tid / F4, sc = (tid % F4) * 4;
    constexpr int RS = NT / F4;  // rows per staging pass (8)
    static_assert(RS == 8 && RTT_T % RS == 0 && RTT_E % RS == 0, "staging map");
    constexpr int TA = RTT_T / 8, TP = RT_PAIRS / NT;  // tokens per lane, pairs per thread
    static_assert(TP >= 1 && RT_PAIRS % NT == 0, "pairs per thread");
    float tot[TP];                    // pairs tid + NT j: token p / 32, expert p % 32
#pragma unroll
    for (int j = 0; j < TP; j++) tot[j] = 0.0f;
    const int G = H / RG, nst = G / CH;
    float4 xv[RTT_T / RS], wv[RTT_E / RS];
    auto fetch = [&](int st) {
        const size_t col = (size_t)st * CH * RG + sc;
#pragma unroll
        for (int v = 0; v < RTT_T / RS; v++) {
            const int t = t0 + sr + RS * v;
            xv[v] = t < T ? *reinterpret_cast<const float4 *>(x + (size_t)t * H + col) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int v = 0; v < RTT_E / RS; v++) {
            const int e = e0 + sr + RS * v;
            wv[v] = e < E ? *reinterpret_cast<const float4 *>(Wr + (size_t)e * H + col) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    fetch(0);
    for (int st = 0; st < nst; st++) {
#pragma unroll
        for (int v = 0; v < RTT_T / RS; v++) *reinterpret_cast<float4 *>(&xs[sr + RS * v][sc]) = xv[v];
#pragma unroll
        for (int v = 0; v < RTT_E / RS; v++) *reinterpret_cast<float4 *>(&ws[sr + RS * v][sc]) = wv[v];
        __syncthreads();  // staged rows in; the previous step's chains read
        if (st + 1 < nst) fetch(st + 1);
        const int gl = gw;
        float a[TA][4];
#pragma unroll
        for (int i = 0; i < TA; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) a[i][j] = 0.0f;
#pragma unroll
        for (int q = 0; q < RG / 4; q++) {
            const int c = gl * RG + 4 * q;
            float xe[TA][4], we[4][4];
#pragma unroll
            for (int i = 0; i < TA; i++) {
                const float4 v = *reinterpret_cast<const float4 *>(&xs[ti + 8 * i][c]);
                xe[i][0] = v.x; xe[i][1] = v.y; xe[i][2] = v.z; xe[i][3] = v.w;
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float4 v = *reinterpret_cast<const float4 *>(&ws[ej + 8 * j][c]);
                we[j][0] = v.x; we[j][1] = v.y; we[j][2] = v.z; we[j][3] = v.w;
            }
#pragma unroll
            for (int cc = 0; cc < 4; cc++)
#pragma unroll
                for (int i = 0; i < TA; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) a[i][j] = __builtin_fmaf(we[j][cc], xe[i][cc], a[i][j]);
        }
#pragma unroll
        for (int i = 0; i < TA; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) cs[gl][(ti + 8 * i) * RTT_E + ej + 8 * j] = a[i][j];
        __syncthreads();  // the step's chains in
#pragma unroll
        for (int j = 0; j < TP; j++)
#pragma unroll
            for (int g = 0; g < CH; g++) tot[j] = tot[j] + cs[g][tid + NT * j];
    }
#pragma unroll
    for (int j = 0; j < TP; j++) {
        const int p = tid + NT * j, t = t0 + p / RTT_E, e = e0 + p % RTT_E;
        if (t < T && e < E) raw[(size_t)t * E + e] = tot[j];
    }
}

// NaN logits rank below every number (as -inf) and -0 equals +0, so the
// 64-bit key orders experts by (logit descending, index ascending) and the
// ranks always form a permutation.
TG_DEV uint64_t rank_key(float l, int e) {
    float v = l != l ? -__builtin_inff() : l;
    v = v + 0.0f;
    uint32_t u = __float_as_uint(v);
    uint32_t mono = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)mono << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)e);
}

// Routing of one token by a 256-thread block, the first thing k_gateup and
// k_topk do.  x -> registers xv (8 per thread per pass) and LDS xf; s ->
// sred[0]; logits -> slog; the top-k expert ids -> sidx[0..k) (descending
// logit, equal logits lower index first).  Ends with a barrier.
constexpr int RO_THREADS = 256;
constexpr int RO_MAXPASS = 4;  // H <= 4 * 8 * 256

// Token t's x into registers: thread tid holds elements ps * 2048 + 8 tid ..
// + 7 of pass ps (zeros past H).
template <int NP = RO_MAXPASS>
TG_DEV void route_x_load(const float *__restrict__ xt, int H, float (&xv)[NP][8]) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int ps = 0; ps < NP; ps++) {
        const int i0 = ps * RO_THREADS * 8 + tid * 8;
        if (i0 < H) {
            const float4 a = *reinterpret_cast<const float4 *>(xt + i0);
            const float4 b = *reinterpret_cast<const float4 *>(xt + i0 + 4);
            xv[ps][0] = a.x; xv[ps][1] = a.y; xv[ps][2] = a.z; xv[ps][3] = a.w;
            xv[ps][4] = b.x; xv[ps][5] = b.y; xv[ps][6] = b.z; xv[ps][7] = b.w;
        } else {
#pragma unroll
            for (int c = 0; c < 8; c++) xv[ps][c] = 0.0f;
        }
    }
}

// xt null: x already in xv (route_x_load); rawt null: this thread's raw dot
// already in r_in (thread e < E: expert e)
template <int NP = RO_MAXPASS>
TG_DEV void route_token(const float *__restrict__ xt, const float *__restrict__ rawt, int E, int H, int k,
                        float eps, float (&xv)[NP][8], float *xf, float *gss, float *slog, uint64_t *keys,
                        int *sidx, float *sred, float r_in = 0.0f) {
    const int tid = threadIdx.x, G = H / RG;
    if (xt) route_x_load<NP>(xt, H, xv);
#pragma unroll
    for (int ps = 0; ps < NP; ps++) {
        const int i0 = ps * RO_THREADS * 8 + tid * 8;
        if (i0 < H) {
            *reinterpret_cast<float4 *>(xf + i0) = make_float4(xv[ps][0], xv[ps][1], xv[ps][2], xv[ps][3]);
            *reinterpret_cast<float4 *>(xf + i0 + 4) = make_float4(xv[ps][4], xv[ps][5], xv[ps][6], xv[ps][7]);
        }
    }
    float r = rawt ? (tid < E ? rawt[tid] : 0.0f) : r_in;
    if (tid < k) sidx[tid] = 0;
    __syncthreads();
    if (tid < G) {
        const float4 *x4 = reinterpret_cast<const float4 *>(xf + tid * RG);
        float a = 0.0f;
#pragma unroll
        for (int q = 0; q < RG / 4; q++) {
            float4 v = x4[q];
            a = __builtin_fmaf(v.x, v.x, a);
            a = __builtin_fmaf(v.y, v.y, a);
            a = __builtin_fmaf(v.z, v.z, a);
            a = __builtin_fmaf(v.w, v.w, a);
        }
        gss[tid] = a;
    }
    __syncthreads();
    if (tid == 0) {  // in ascending group order; the values read 32 at a time, ahead of their adds
        float tot = 0.0f;
        if ((G & 3) == 0) {
            const float4 *g4 = reinterpret_cast<const float4 *>(gss);
            for (int q0 = 0; q0 < G / 4; q0 += 8) {
                float4 v[8];
#pragma unroll
                for (int q = 0; q < 8; q++) v[q] = g4[min(q0 + q, G / 4 - 1)];
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    if (q0 + q < G / 4) {
                        tot = tot + v[q].x;
                        tot = tot + v[q].y;
                        tot = tot + v[q].z;
                        tot = tot + v[q].w;
                    }
                }
            }
        } else {
            for (int g = 0; g < G; g++) tot = tot + gss[g];
        }
        sred[0] = rms_scale(tot, H, eps);
    }
    __syncthreads();
    if (tid < E) {
        float l = r * sred[0];
        slog[tid] = l;
        keys[tid] = rank_key(l, tid);
    }
    __syncthreads();
    // rank = number of larger keys; two threads per expert when E <= 128
    const int tpe = 2 * E <= RO_THREADS ? 2 : 1;
    const int e = tpe == 2 ? tid >> 1 : tid;
    if (e < E) {
        const uint64_t my = keys[e];
        int half = tpe == 2 ? (tid & 1) : 0;
        int n = E / tpe, b0 = half * n;
        int cnt = 0;
#pragma unroll 8
        for (int i = 0; i < n; i += 2) {
            ulonglong2 o = *reinterpret_cast<const ulonglong2 *>(keys + b0 + i);
            cnt += o.x > my ? 1 : 0;
            cnt += o.y > my ? 1 : 0;
        }
        if (tpe == 2) cnt += __shfl_xor(cnt, 1, WAVE);
        if (half == 0 && cnt < k) sidx[cnt] = e;
    }
    __syncthreads();
}

// Renormalised softmax over the selected logits (engine.py:233-236): the k
// values in ascending order, e = exp(l - lmax), numpy's pairwise sum, w = e /
// sum.  One thread.
TG_DEV void topk_softmax(const float *slog, const int *sidx, int k, float *sw, float *sex) {
    float lmax = slog[sidx[0]];
    for (int i = 0; i < k; i++) sex[i] = expf_tg(slog[sidx[k - 1 - i]] - lmax);
    float sum = np_pairwise_sum(sex, k);
    for (int i = 0; i < k; i++) sw[k - 1 - i] = sex[i] / sum;
}

struct RouteLds {
    float *xf, *gss, *slog, *sw, *sex, *sred;
    uint64_t *keys;
    int *sidx;
};

// LDS for route_token: xf[H] gss[256] slog[MAX_E] sw/sex[MAX_K] sred[4]
// keys[MAX_E] sidx[MAX_K], from a 16-byte aligned base.
__host__ __device__ inline size_t route_lds_bytes(int H) {
    return 4 * (size_t)H + 4 * 256 + 4 * MAX_E + 8 * MAX_K + 16 + 8 * MAX_E + 4 * MAX_K;
}

TG_DEV RouteLds route_lds(uint8_t *base, int H) {
    RouteLds r;
    r.keys = reinterpret_cast<uint64_t *>(base);
    r.xf = reinterpret_cast<float *>(r.keys + MAX_E);
    r.gss = r.xf + H;
    r.slog = r.gss + 256;
    r.sw = r.slog + MAX_E;
    r.sex = r.sw + MAX_K;
    r.sred = r.sex + MAX_K;
    r.sidx = reinterpret_cast<int *>(r.sred + 4);
    return r;
}

// Grid (T): logits, top-k and weights (tg_router_topk_dev).
__global__ __launch_bounds__(RO_THREADS) void k_topk(const float *__restrict__ raw, const float *__restrict__ x, int E,
                                                     int H, int k, float eps, float *__restrict__ logits,
                                                     int32_t *__restrict__ idx, float *__restrict__ w) {
    extern __shared__ __align__(16) uint8_t smem[];
    RouteLds L = route_lds(smem, H);
    const int t = blockIdx.x;
    float xv[RO_MAXPASS][8];
    route_token(x + (size_t)t * H, raw + (size_t)t * E, E, H, k, eps, xv, L.xf, L.gss, L.slog, L.keys, L.sidx,
                L.sred);
    for (int e = threadIdx.x; e < E; e += blockDim.x) logits[(size_t)t * E + e] = L.slog[e];
    if (threadIdx.x == 0) {
        topk_softmax(L.slog, L.sidx, k, L.sw, L.sex);
        for (int i = 0; i < k; i++) {
            if (idx) idx[(size_t)t * k + i] = L.sidx[i];
            if (w) w[(size_t)t * k + i] = L.sw[i];
        }
    }
}

// ================================================================ Q8_0
// Q8_0 of 8 values held by this thread; 4 consecutive threads form one block
// of 32.  Writes the LDS activation form (qs, float(half d), block sum).
TG_DEV void q8_group8(const float *v, bool on, int i0, int8_t *qs, float *dsc, int *sum) {
    float a = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; c++) a = fabsf(v[c]) > a ? fabsf(v[c]) : a;
    float o = __shfl_xor(a, 1, WAVE);
    a = o > a ? o : a;
    o = __shfl_xor(a, 2, WAVE);
    a = o > a ? o : a;
    float d = a / 127.0f;
    float inv = a > 0.0f ? 127.0f / a : 0.0f;
    int q[8], qsum = 0;
#pragma unroll
    for (int c = 0; c < 8; c++) {
        q[c] = (int)__builtin_rintf(v[c] * inv);
        qsum += q[c];
    }
    qsum += __shfl_xor(qsum, 1, WAVE);
    qsum += __shfl_xor(qsum, 2, WAVE);
    if (on) {
        uint32_t lo = (uint32_t)(q[0] & 255) | ((uint32_t)(q[1] & 255) << 8) | ((uint32_t)(q[2] & 255) << 16) |
                      ((uint32_t)(q[3] & 255) << 24);
        uint32_t hi = (uint32_t)(q[4] & 255) | ((uint32_t)(q[5] & 255) << 8) | ((uint32_t)(q[6] & 255) << 16) |
                      ((uint32_t)(q[7] & 255) << 24);
        *reinterpret_cast<uint2 *>(qs + i0) = make_uint2(lo, hi);
        if ((i0 & 31) == 0) {
            dsc[i0 >> 5] = h2f(f2h(d));
            sum[i0 >> 5] = qsum;
        }
    }
}

// Weighted combine of one output row over the k slots, acc = fma(w_j, D_j,
// acc) for j = k-1 .. 0 (ascending logit order): D_j = D[j * stride + r],
// both operands read from LDS eight slots per round before the fmas.
TG_DEV float combine_slots(const float *sw, const float *D, int stride, int k, int r) {
    float acc = 0.0f;
    for (int c = k - 1; c >= 0; c -= 8) {
        float dd[8], ww[8];
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int j = c - q < 0 ? 0 : c - q;
            dd[q] = D[j * stride + r];
            ww[q] = sw[j];
        }
#pragma unroll
        for (int q = 0; q < 8; q++)
            if (c - q >= 0) acc = __builtin_fmaf(ww[q], dd[q], acc);
    }
    return acc;
}

// Sequential row accumulation acc = fma(U_b, dx_b, acc), operands read from
// LDS four at a time (U and dx 16-byte aligned).
TG_DEV float chain4(const float *U, const float *dx, int nb) {
    float acc = 0.0f;
    const float4 *u4 = reinterpret_cast<const float4 *>(U);
    const float4 *d4 = reinterpret_cast<const float4 *>(dx);
    int q = 0;
#pragma unroll 4
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

__host__ __device__ inline int round4(int n) { return (n + 3) & ~3; }

// ============================================================ decode routing
// Block (e, t): the raw router dot of expert e for token t (grouped sums as
// k_route) and, from the same x, the token's RMS scale s (grouped sums of
// squares as route_token), so logit = raw * s as in route_token.  Thread 0
// publishes the logit as a tagged word (relaxed agent-scope atomics).  Block (0, t) also ranks the token: it forms
// Q8_0(x * s), reads the E logits (bounded polls on the tags), ranks them,
// forms the softmax weights, and writes idx / w / xq / xd / xs for the
// expert kernels.
//
// ctl[2t+1] is the generation of the token's last routing (ctl[2t] is
// unused).  A launch publishes with the next generation, so words left by
// earlier launches never match; block (0, t) stores the new generation,
// which the next launch reads (after the kernel boundary).  A poll that
// runs out of tries sets *err and routes the token to experts 0..k-1 with
// weight 0, so the expert kernels stay in bounds.
constexpr uint32_t RD_SPIN_LIMIT = 1u << 20;
constexpr int RD_THREADS = 1024;  // several threads per expert in the ranking

// Failure-channel test hook (set_fault_injection): the poll bound of the
// one-token expert launches (k_experts, k_layer_dec) and one h line whose
// publication they leave out, so that every reader's bounded wait runs out
// while each kernel still exits normally.  0 / -1 in normal use.
static uint32_t g_fault_spin = 0;
static int g_fault_drop = -1;

static uint32_t fault_spin_limit() { return g_fault_spin ? g_fault_spin : RD_SPIN_LIMIT; }
uint32_t poll_spin_limit() { return fault_spin_limit(); }
int poll_drop() { return g_fault_drop; }

void set_fault_injection(uint32_t spin_limit, int drop_line) {
    g_fault_spin = spin_limit;
    g_fault_drop = drop_line < 0 ? -1 : drop_line;
}

TG_DEV uint32_t next_gen(uint32_t g) { return g >= 0x7FFFFFFFu ? 1u : g + 1u; }

// Top-k of E ranked keys (LDS) by a block of RD_THREADS threads: rank =
// number of larger keys; sidx[rank] = expert for rank < k.  Thread t takes
// expert t % EW (EW = E rounded up to a whole number of waves) against
// slice t / EW of the keys, so all lanes of a wave read the same keys
// (LDS broadcast); the slice counts meet in rcnt[] (LDS, zero on entry) by
// LDS atomics.  Ends with a barrier.
TG_DEV void rank_topk(const uint64_t *keys, int E, int k, int *sidx, int *rcnt) {
    const int tid = threadIdx.x;
    // per-wave (scalar) slice arithmetic: a wave lies in one slice
    const int ewv = (E + WAVE - 1) / WAVE, parts = (RD_THREADS / WAVE) / ewv;
    const int wv = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int part = wv / ewv, e = tid - part * ewv * WAVE;
    if (e < E && part < parts) {
        const uint64_t my = keys[e];
        const int b0 = part * E / parts, b1 = (part + 1) * E / parts;
        int cnt = 0;
        for (int c = b0; c < b1; c += 8) {  // 8 keys loaded per round, then compared
            uint64_t kk[8];
#pragma unroll
            for (int q = 0; q < 8; q++) kk[q] = keys[min(c + q, b1 - 1)];
#pragma unroll
            for (int q = 0; q < 8; q++) cnt += (c + q < b1 && kk[q] > my) ? 1 : 0;
        }
        if (cnt) atomicAdd(rcnt + e, cnt);
    }
    __syncthreads();
    if (tid < E && rcnt[tid] < k) sidx[rcnt[tid]] = tid;
    __syncthreads();
}

// Renormalised softmax over the selected logits (engine.py:233-236) by one
// wave, lane i < k holding slot j = k-1-i: e_i = exp(l - lmax) in
// ascending order, numpy's pairwise sum, returns w_j = e / sum (lanes >= k
// return 0).
TG_DEV float topk_softmax_lane(const float *slog, const int *sidx, int k) {
    const int lane = threadIdx.x & (WAVE - 1);
    const float lmax = slog[sidx[0]];
    const bool on = lane < k;
    const float ex = on ? expf_tg(slog[sidx[on ? k - 1 - lane : 0]] - lmax) : 0.0f;
    float sex[MAX_K];
#pragma unroll
    for (int i = 0; i < MAX_K; i++) sex[i] = __shfl(ex, i, WAVE);
    const float sum = np_pairwise_sum(sex, k);
    return on ? ex / sum : 0.0f;
}

__global__ __launch_bounds__(RD_THREADS) void k_route_dec(const float *__restrict__ Wr, const float *__restrict__ x,
                                                          const float *__restrict__ gn, int E, int H, int k, float eps,
                                                          uint64_t *__restrict__ lw,
                                                          uint32_t *__restrict__ ctl, uint32_t *__restrict__ err,
                                                          int32_t *__restrict__ idx, float *__restrict__ w,
                                                          int8_t *__restrict__ xq, float *__restrict__ xd,
                                                          int *__restrict__ xs) {
    __shared__ __align__(16) float gp[RT_THREADS];
    __shared__ __align__(16) float gq[RT_THREADS];
    __shared__ __align__(16) uint64_t keys[MAX_E];
    __shared__ int rcnt[MAX_E];
    __shared__ float slog[MAX_E];
    __shared__ int sidx[MAX_K];
    __shared__ float ssc;
    __shared__ int bad;
    const int e = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, G = H / RG, nbH = H / QK;
    const float *xt = x + (size_t)t * H;
    const uint32_t tag = next_gen(__hip_atomic_load(ctl + 2 * t + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    if (tid < G) {
        const float4 *w4 = reinterpret_cast<const float4 *>(Wr + (size_t)e * H + tid * RG);
        const float4 *x4 = reinterpret_cast<const float4 *>(xt + tid * RG);
        float4 wv[RG / 4], xv[RG / 4];
#pragma unroll
        for (int q = 0; q < RG / 4; q++) {
            wv[q] = w4[q];
            xv[q] = x4[q];
        }
        float aw = 0.0f, aq = 0.0f;
#pragma unroll
        for (int q = 0; q < RG / 4; q++) {
            aq = __builtin_fmaf(xv[q].x, xv[q].x, aq);
            aq = __builtin_fmaf(xv[q].y, xv[q].y, aq);
            aq = __builtin_fmaf(xv[q].z, xv[q].z, aq);
            aq = __builtin_fmaf(xv[q].w, xv[q].w, aq);
        }
#pragma unroll
        for (int q = 0; q < RG / 4; q++) {
            aw = __builtin_fmaf(wv[q].x, xv[q].x, aw);
            aw = __builtin_fmaf(wv[q].y, xv[q].y, aw);
            aw = __builtin_fmaf(wv[q].z, xv[q].z, aw);
            aw = __builtin_fmaf(wv[q].w, xv[q].w, aw);
        }
        gp[tid] = aw;
        gq[tid] = aq;
    }
    if (tid == 0) bad = 0;
    __syncthreads();
    if (tid == 0) {
        // both totals in ascending group order (G is a multiple of 8)
        const float4 *p4 = reinterpret_cast<const float4 *>(gp);
        const float4 *q4 = reinterpret_cast<const float4 *>(gq);
        float tr = 0.0f, ts = 0.0f;
#pragma unroll 4
        for (int g = 0; g < G / 4; g++) {
            const float4 a = p4[g], b = q4[g];
            tr = tr + a.x; tr = tr + a.y; tr = tr + a.z; tr = tr + a.w;
            ts = ts + b.x; ts = ts + b.y; ts = ts + b.z; ts = ts + b.w;
        }
        const float sc = rms_scale(ts, H, eps);
        ll_put(lw + (size_t)t * E + e, __float_as_uint(tr * sc), tag);
        ssc = sc;
    }
    if (e != 0) return;
    __syncthreads();

    // ---- block (0, t): Q8_0((x * s) * g), then the E logits
    const float sc = ssc;
    {
        const int i0 = tid * 8;
        if (i0 < H) {  // H / 8 is a multiple of 32: whole 4-lane groups
            const float4 a4 = *reinterpret_cast<const float4 *>(xt + i0);
            const float4 b4 = *reinterpret_cast<const float4 *>(xt + i0 + 4);
            const float4 ga = *reinterpret_cast<const float4 *>(gn + i0);
            const float4 gb = *reinterpret_cast<const float4 *>(gn + i0 + 4);
            const float v[8] = {(a4.x * sc) * ga.x, (a4.y * sc) * ga.y, (a4.z * sc) * ga.z, (a4.w * sc) * ga.w,
                                (b4.x * sc) * gb.x, (b4.y * sc) * gb.y, (b4.z * sc) * gb.z, (b4.w * sc) * gb.w};
            q8_group8(v, true, i0, xq + (size_t)t * H, xd + (size_t)t * nbH, xs + (size_t)t * nbH);
        }
    }
    if (tid < k) sidx[tid] = 0;
    if (tid < E) {
        const uint64_t *src = lw + (size_t)t * E + tid;
        uint64_t v = ll_get(src);
        uint32_t tries = 0;
        while ((uint32_t)(v >> 32) != tag) {
            if (++tries >= RD_SPIN_LIMIT) {
                bad = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            v = ll_get(src);
        }
        const float l = __uint_as_float((uint32_t)v);
        slog[tid] = l;
        keys[tid] = rank_key(l, tid);
        rcnt[tid] = 0;
    }
    __syncthreads();
    rank_topk(keys, E, k, sidx, rcnt);
    if (tid < WAVE) {
        const float wj = topk_softmax_lane(slog, sidx, k);
        if (tid < k) {
            const int j = k - 1 - tid;
            idx[(size_t)t * k + j] = bad ? j : sidx[j];
            w[(size_t)t * k + j] = bad ? 0.0f : wj;
        }
    }
    if (tid == 0) {
        if (bad) __hip_atomic_store(err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(ctl + 2 * t + 1, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ============================================================ gate / up
// Block (m, j, t): rows [32m, 32m+32) of gate and of up of token t's j-th
// selected expert against Q8_0(x_t * s_t), h = SiLU(gate) * up, and the
// Q8_0 block m of h.  The nibble loads are issued right after the expert id
// is read; thread p of the block owns the row-block items p + u * 1024.
constexpr int GU_THREADS = 1024;
constexpr int GU_ROWS = 32;  // one Q8_0 block of h

__host__ __device__ inline size_t gateup_lds_bytes(int H, int nbH) {
    // xq[H] | xd[r4] | xs[r4] | U[2 * 32 * (r4 + 4)] | accs[64]
    return (size_t)H + 8 * (size_t)round4(nbH) + 4 * (size_t)2 * GU_ROWS * (round4(nbH) + 4) + 4 * 2 * GU_ROWS;
}

template <int UNR>
__global__ __launch_bounds__(GU_THREADS) void k_gateup(const uint8_t *__restrict__ layer_pl, Shape s,
                                                       const int32_t *__restrict__ idx,
                                                       const int8_t *__restrict__ xq_g,
                                                       const float *__restrict__ xd_g, const int *__restrict__ xs_g,
                                                       int8_t *__restrict__ hq, float *__restrict__ hd,
                                                       int *__restrict__ hs) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int RT = GU_ROWS;
    const int nb = s.nbH, ust = round4(nb) + 4, H = s.H, I = s.I, tid = threadIdx.x;
    int8_t *xq = reinterpret_cast<int8_t *>(smem);
    float *xd = reinterpret_cast<float *>(xq + H);
    int *xs = reinterpret_cast<int *>(xd + round4(nb));
    float *U = reinterpret_cast<float *>(xs + round4(nb));
    float *accs = U + 2 * RT * ust;
    const int m = blockIdx.x, j = blockIdx.y, t = blockIdx.z, r0 = m * RT;
    const size_t slot = (size_t)t * s.k + j;
    int e = idx[slot];
    e = e < 0 ? 0 : (e >= s.E ? s.E - 1 : e);  // never address outside the layer
    const uint8_t *ex = layer_pl + (size_t)e * s.EB;
    const size_t ntb = (size_t)I * nb;
    const int items = 2 * RT * nb;
    // every thread loads (items past the end clamped to the last, unused):
    // no branch between the loads, so all are in flight before the first wait
    uint4 wv[UNR];
    uint32_t dv[UNR];
#pragma unroll
    for (int u = 0; u < UNR; u++) {
        const int p = min(u * GU_THREADS + tid, items - 1);
        const int rd = (int)fdiv((uint32_t)p, s.divH), b = p - rd * nb;
        const int mat = rd >= RT ? 1 : 0;
        const uint8_t *tb = ex + (size_t)mat * s.GB;
        const size_t o = (size_t)(r0 + rd - mat * RT) * nb + b;
        wv[u] = reinterpret_cast<const uint4 *>(tb)[o];
        dv[u] = reinterpret_cast<const uint16_t *>(tb + ntb * 16)[o];
    }
    if (tid < H / 8) reinterpret_cast<uint2 *>(xq)[tid] = reinterpret_cast<const uint2 *>(xq_g + (size_t)t * H)[tid];
    if (tid < nb) {
        xd[tid] = xd_g[(size_t)t * nb + tid];
        xs[tid] = xs_g[(size_t)t * nb + tid];
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < UNR; u++) {
        const int p = u * GU_THREADS + tid;
        if (p < items) {
            const int rd = (int)fdiv((uint32_t)p, s.divH), b = p - rd * nb;
            const int S = dot_q4_q8(wv[u], reinterpret_cast<const int *>(xq + b * QK)) - 8 * xs[b];
            U[rd * ust + b] = (float)S * h2f(dv[u]);
        }
    }
    __syncthreads();
    if (tid < 2 * RT) accs[tid] = chain4(U + tid * ust, xd, nb);
    __syncthreads();
    if (tid < 64) {  // wave 0; both halves compute, the first writes
        const int i = tid & 31;
        const float hv = silu_mul(accs[i], accs[RT + i]);
        float dq;
        int qsum;
        uint16_t dh;
        const int q = q8_lane(hv, dq, qsum, dh);
        if (tid < 32) {
            hq[slot * I + r0 + i] = (int8_t)q;
            if (i == 0) {
                hd[slot * s.nbI + m] = dq;
                hs[slot * s.nbI + m] = qsum;
            }
        }
    }
}

// ============================================================ down
// Block (g, t): rows [g*RD, g*RD+RD) of down for the k experts of token t
// against their Q8_0 h, combined: out = sum_j w_j down_j in ascending logit
// order (j = k-1 .. 0) plus resid when given.  The nibble loads are issued
// before h is staged in LDS.
constexpr int DN_RD = 8;
constexpr int DN_THREADS = 256;

__host__ __device__ inline size_t down_lds_bytes(int k, int I, int nbI) {
    // hq[k*I] | hd[k*r4] | hs[k*r4] | U[k*RD*(r4+4)] | D[k*RD] | sw[MAX_K] | sidx[MAX_K]
    return (size_t)k * I + 8 * (size_t)k * round4(nbI) + 4 * (size_t)k * DN_RD * (round4(nbI) + 4) +
           4 * (size_t)k * DN_RD + 8 * MAX_K;
}

template <int UNR>
__global__ __launch_bounds__(DN_THREADS) void k_down(const uint8_t *__restrict__ layer_pl, Shape s,
                                                     const int32_t *__restrict__ idx, const float *__restrict__ w,
                                                     const int8_t *__restrict__ hq_g, const float *__restrict__ hd_g,
                                                     const int *__restrict__ hs_g, const float *resid, float *out) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int RD = DN_RD, lrd = 3;  // RD = 2^lrd
    static_assert(RD == 1 << lrd, "down rows per block");
    const int k = s.k, nb = s.nbI, nbp = round4(nb), I = s.I, H = s.H, ust = round4(nb) + 4;
    const int tid = threadIdx.x;
    int8_t *hq = reinterpret_cast<int8_t *>(smem);
    float *hd = reinterpret_cast<float *>(smem + (size_t)k * I);
    int *hs = reinterpret_cast<int *>(hd + k * nbp);
    float *U = reinterpret_cast<float *>(hs + k * nbp);
    float *D = U + k * RD * ust;
    float *sw = D + k * RD;
    int *sidx = reinterpret_cast<int *>(sw + MAX_K);

    const int t = blockIdx.y, r0 = blockIdx.x * RD;
    if (tid < k) {
        const int e = idx[(size_t)t * k + tid];
        sidx[tid] = e < 0 ? 0 : (e >= s.E ? s.E - 1 : e);  // never address outside the layer
        sw[tid] = w[(size_t)t * k + tid];
    }
    float rv = 0.0f;
    if (resid && tid < RD) rv = resid[(size_t)t * H + r0 + tid];
    __syncthreads();

    const size_t ntb = (size_t)H * nb;
    const int items = k * RD * nb;
    uint4 wv[UNR];
    uint32_t dv[UNR];
#pragma unroll
    for (int u = 0; u < UNR; u++) {  // clamped, unbranched loads (as k_gateup)
        const int p = min(u * DN_THREADS + tid, items - 1);
        const int rd = (int)fdiv((uint32_t)p, s.divI), b = p - rd * nb;
        const int jj = rd >> lrd, row = r0 + (rd - (jj << lrd));
        const uint8_t *tb = layer_pl + (size_t)sidx[jj] * s.EB + 2 * s.GB;
        const size_t o = (size_t)row * nb + b;
        wv[u] = reinterpret_cast<const uint4 *>(tb)[o];
        dv[u] = reinterpret_cast<const uint16_t *>(tb + ntb * 16)[o];
    }
    // the token's Q8_0 h: k * I bytes, k * nbI scales and sums
    const size_t hbase = (size_t)t * k;
    const uint4 *hq4 = reinterpret_cast<const uint4 *>(hq_g + hbase * I);
    for (int i = tid; i < k * I / 16; i += DN_THREADS) reinterpret_cast<uint4 *>(hq)[i] = hq4[i];
    for (int i = tid; i < k * nb; i += DN_THREADS) {
        const int jj = i / nb, b = i - jj * nb;
        hd[jj * nbp + b] = hd_g[hbase * nb + i];
        hs[jj * nbp + b] = hs_g[hbase * nb + i];
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < UNR; u++) {
        const int p = u * DN_THREADS + tid;
        if (p < items) {
            const int rd = (int)fdiv((uint32_t)p, s.divI), b = p - rd * nb;
            const int jj = rd >> lrd;
            const int S = dot_q4_q8(wv[u], reinterpret_cast<const int *>(hq + (size_t)jj * I + b * QK)) -
                          8 * hs[jj * nbp + b];
            U[rd * ust + b] = (float)S * h2f(dv[u]);
        }
    }
    __syncthreads();
    for (int rd = tid; rd < k * RD; rd += DN_THREADS) D[rd] = chain4(U + rd * ust, hd + (rd / RD) * nbp, nb);
    __syncthreads();
    if (tid < RD) {
        const float acc = combine_slots(sw, D, RD, k, tid);
        out[(size_t)t * H + r0 + tid] = resid ? rv + acc : acc;
    }
}

// ============================================================ fused experts (one token)
// One launch per layer for gate/up and down of a single token, so the down
// weights stream while gate/up runs instead of after it.  The grid has one
// block of 1024 threads per down unit (H / RD units of RD output rows, at
// most one block per CU, so every block is resident at once).  Block b:
//   1. runs its first gate/up unit (unit (m, j): rows [32m, 32m+32) of gate
//      and up of the j-th expert, as k_gateup), wave 0 publishing the Q8_0
//      block of h as FX_QW tagged words;
//   2. issues, from waves 3.., the loads of its down unit (RD rows of down
//      for all k experts), then runs any further gate/up units;
//   3. waves 0..2 read the FX_QW words of every unit (thread u: unit u; a
//      unit's words fill one 128-byte line of their own, written by one
//      store; the last word polled with coherent loads, the rest read
//      through the L2), then waves 3.. dot the down rows and the block chains,
//      combines and adds the residual for its RD rows.  The reading waves
//      hold no down load, so their waits (vmcnt retires in order) never
//      stand behind the down stream.
// Tags: the routing generation of the layer (ctl[1], stored by k_route_dec
// of the same layer), so words of earlier layers never match.  A block finishes its own gate/up units
// before it waits, so no wait depends on a block that is not running.
// Polls are bounded; when one runs out the block sets *err and writes NaN
// rows.
constexpr int FX_THREADS = 1024;
constexpr int FX_PT = 3 * WAVE;              // threads that poll the h words (waves 0..2)
constexpr int FX_DT = FX_THREADS - FX_PT;    // threads that load and dot the down rows
constexpr int FX_QW = 10;                    // tagged words per unit of h
constexpr int FX_QS = 16;                    // word stride of the units (one 128-byte line each)

struct FxArgs {
    const uint8_t *layer_pl;
    const int32_t *idx;
    const float *w;
    const int8_t *xq;
    const float *xd;
    const int *xs;
    uint64_t *hw;         // [2][k * I/32][FX_QS] tagged h blocks, by tag parity
    const uint32_t *ctl;  // routing counter / generation of token 0
    uint32_t *err;
    const float *resid;
    float *out;
    int rd;               // down rows per block (grid = H / rd)
    uint32_t spin;        // poll bound (fault_spin_limit())
    int drop;             // h line left unpublished (-1 in normal use)
};

__host__ __device__ inline size_t fx_down_lds_bytes(int k, int I, int nbI, int rd) {
    // hq[k*I] | hd[k*r4] | hs[k*r4] | U[k*rd*(r4+4)] | D[k*rd]
    return (size_t)k * I + 8 * (size_t)k * round4(nbI) + 4 * (size_t)k * rd * (round4(nbI) + 4) +
           4 * (size_t)k * rd;
}

// The down part sits after the gate/up part: the reading waves fill it while
// wave 0 may still be publishing the block's last unit from the gate/up part.
__host__ __device__ inline size_t fx_down_off(const Shape &s) { return (gateup_lds_bytes(s.H, s.nbH) + 15) & ~(size_t)15; }

__host__ __device__ inline size_t fx_lds_bytes(const Shape &s, int rd) {
    return fx_down_off(s) + fx_down_lds_bytes(s.k, s.I, s.nbI, rd);
}

// Gate/up unit (m, j) in three steps, so a block can issue its down loads
// between the dots and the rest: the nibble and scale loads of rows
// [32m, 32m+32) of gate and up of the j-th expert ...
template <int UG>
struct FxGu {
    uint4 wv[UG];
    uint32_t dv[UG];
};

// Marks every register of a unit's loads as read (an empty asm taking them
// all), after its dots: the dots skip clamped items, so without this the
// compiler keeps such loads pending and waits for them when it reuses
// their registers, which can land behind later loads.
template <int UG>
TG_DEV void fx_consume(const FxGu<UG> &g) {
#pragma unroll
    for (int i = 0; i < UG; i++) __asm__ volatile("" ::"v"(g.wv[i].x), "v"(g.wv[i].y), "v"(g.wv[i].z), "v"(g.wv[i].w), "v"(g.dv[i]));
}

// (eid: the block's clamped expert ids by slot, in LDS)
template <int UG>
TG_DEV void fx_gu_load(const uint8_t *layer_pl, const Shape &s, int unit, const int *eid, FxGu<UG> &g) {
    constexpr int RT = GU_ROWS;
    const int nb = s.nbH, I = s.I, tid = threadIdx.x;
    const int mI = I / RT, m = unit % mI, j = unit / mI, r0 = m * RT;
    const uint8_t *ex = layer_pl + (size_t)eid[j] * s.EB;
    const size_t ntb = (size_t)I * nb;
    const int items = 2 * RT * nb;
#pragma unroll
    for (int u = 0; u < UG; u++) {  // clamped, unbranched loads (as k_gateup)
        const int p = min(u * FX_THREADS + tid, items - 1);
        const int rd = (int)fdiv((uint32_t)p, s.divH), b = p - rd * nb;
        const int mat = rd >= RT ? 1 : 0;
        const uint8_t *tb = ex + (size_t)mat * s.GB;
        const size_t o = (size_t)(r0 + rd - mat * RT) * nb + b;
        g.wv[u] = reinterpret_cast<const uint4 *>(tb)[o];
        g.dv[u] = reinterpret_cast<const uint16_t *>(tb + ntb * 16)[o];
    }
}

// ... the block dots against Q8_0(x * s) into U (LDS; Q8_0 x copied in
// from gxq / gxd / gxs first unless gxq is null, when it is already there) ...
template <int UG>
TG_DEV void fx_gu_dots(const int8_t *gxq, const float *gxd, const int *gxs, const Shape &s, const FxGu<UG> &g,
                       uint8_t *smem) {
    constexpr int RT = GU_ROWS;
    const int nb = s.nbH, ust = round4(nb) + 4, H = s.H, tid = threadIdx.x;
    int8_t *xq = reinterpret_cast<int8_t *>(smem);
    float *xd = reinterpret_cast<float *>(xq + H);
    int *xs = reinterpret_cast<int *>(xd + round4(nb));
    float *U = reinterpret_cast<float *>(xs + round4(nb));
    const int items = 2 * RT * nb;
    if (gxq) {
        if (tid < H / 8) reinterpret_cast<uint2 *>(xq)[tid] = reinterpret_cast<const uint2 *>(gxq)[tid];
        if (tid < nb) {
            xd[tid] = gxd[tid];
            xs[tid] = gxs[tid];
        }
    }
    lds_barrier();  // LDS only: the block's other loads stay in flight
#pragma unroll
    for (int u = 0; u < UG; u++) {
        const int p = u * FX_THREADS + tid;
        if (p < items) {
            const int rd = (int)fdiv((uint32_t)p, s.divH), b = p - rd * nb;
            const int S = dot_q4_q8(g.wv[u], reinterpret_cast<const int *>(xq + b * QK)) - 8 * xs[b];
            U[rd * ust + b] = (float)S * h2f((uint16_t)at_use(g.dv[u]));
        }
    }
    lds_barrier();
}

// ... and the chains, SwiGLU and Q8_0 of the 32 h rows, published as FX_QW
// tagged words.  Wave 0 alone does this part (lane r chains row r: gate
// rows in lanes 0..31, up rows in 32..63) and needs no block barrier, so it
// never waits for the down loads the block has in flight.
TG_DEV void fx_gu_publish(const Shape &s, int unit, uint32_t tag, uint64_t *hw, const uint8_t *smem, int drop) {
    constexpr int RT = GU_ROWS;
    static_assert(2 * RT == 64, "one wave holds the gate and up rows of a unit");
    const int nb = s.nbH, ust = round4(nb) + 4, H = s.H, tid = threadIdx.x;
    const float *xd = reinterpret_cast<const float *>(smem + H);
    const float *U = xd + 2 * round4(nb);
    if (tid < 64) {  // both halves compute the block, lanes 0..9 publish it
        const float a = chain4(U + tid * ust, xd, nb);
        const int i = tid & 31;
        const float hv = silu_mul(__shfl(a, i, WAVE), __shfl(a, i + RT, WAVE));
        float dq;
        int qsum;
        uint16_t dh;
        const int q = q8_lane(hv, dq, qsum, dh);
        const int l4 = 4 * (tid & 7);
        const uint32_t word = (uint32_t)(__shfl(q, l4, WAVE) & 255) | ((uint32_t)(__shfl(q, l4 + 1, WAVE) & 255) << 8) |
                              ((uint32_t)(__shfl(q, l4 + 2, WAVE) & 255) << 16) |
                              ((uint32_t)(__shfl(q, l4 + 3, WAVE) & 255) << 24);
        // lanes 0..7 the packed bytes, 8 the scale, 9 the sum: one store
        const uint32_t pay = tid < 8 ? word : (tid == 8 ? __float_as_uint(dq) : (uint32_t)qsum);
        if (tid < FX_QW && unit != drop) ll_put(hw + (size_t)unit * FX_QS + tid, pay, tag);
    }
}

// Words 0 .. NW-2 of a line whose last word already carries `tag`: plain
// loads (the line holds one unit's words only, written by one store, and is
// shared through the L2 by the blocks of an XCD), then coherent polls of a
// word that still carries an old tag.  Bounded (tries counts on); false
// when a poll ran out of tries.
template <int NW>
TG_DEV bool fx_read_rest(const uint64_t *src, uint32_t tag, uint32_t (&pay)[NW], uint32_t &tries, uint32_t lim) {
    constexpr int LAST = NW - 1;
    __asm__ volatile("" ::: "memory");  // the plain loads stay after the poll
    uint32_t pend = 0;
    uint64_t w[LAST];
#pragma unroll
    for (int i = 0; i < LAST; i++) w[i] = src[i];
#pragma unroll
    for (int i = 0; i < LAST; i++) {
        if ((uint32_t)(w[i] >> 32) == tag)
            pay[i] = (uint32_t)w[i];
        else
            pend |= 1u << i;
    }
    while (pend) {
#pragma unroll
        for (int i = 0; i < LAST; i++)
            if (pend >> i & 1u) w[i] = ll_get(src + i);
#pragma unroll
        for (int i = 0; i < LAST; i++)
            if ((pend >> i & 1u) && (uint32_t)(w[i] >> 32) == tag) {
                pay[i] = (uint32_t)w[i];
                pend &= ~(1u << i);
            }
        if (!pend) break;
        if (++tries >= lim) return false;
        __builtin_amdgcn_s_sleep(2);
    }
    return true;
}

// Reads the NW tagged words of one unit (its line at src): polls the last
// word with coherent loads until it carries `tag`, then the rest as above.
// Bounded; false when a poll ran out of tries.
template <int NW>
TG_DEV bool fx_read_words(const uint64_t *src, uint32_t tag, uint32_t (&pay)[NW], uint32_t lim) {
    constexpr int LAST = NW - 1;
    uint32_t tries = 0;
#pragma unroll
    for (int i = 0; i < NW; i++) pay[i] = 0u;
    uint64_t v = ll_get(src + LAST);
    while ((uint32_t)(v >> 32) != tag) {
        if (++tries >= lim) return false;
        __builtin_amdgcn_s_sleep(2);
        v = ll_get(src + LAST);
    }
    pay[LAST] = (uint32_t)v;
    return fx_read_rest<NW>(src, tag, pay, tries, lim);
}

// The two half-unit lines of one unit: both last words are polled in the
// same rounds (one poll latency for the two lines), then each line's rest.
template <int NW>
TG_DEV bool fx_read_pair(const uint64_t *sa, const uint64_t *sb, uint32_t tag, uint32_t (&pa)[NW],
                         uint32_t (&pb)[NW], uint32_t lim) {
    constexpr int LAST = NW - 1;
    uint32_t tries = 0;
#pragma unroll
    for (int i = 0; i < NW; i++) {
        pa[i] = 0u;
        pb[i] = 0u;
    }
    uint64_t va = ll_get(sa + LAST), vb = ll_get(sb + LAST);
    while ((uint32_t)(va >> 32) != tag || (uint32_t)(vb >> 32) != tag) {
        if (++tries >= lim) return false;
        __builtin_amdgcn_s_sleep(2);
        if ((uint32_t)(va >> 32) != tag) va = ll_get(sa + LAST);
        if ((uint32_t)(vb >> 32) != tag) vb = ll_get(sb + LAST);
    }
    pa[LAST] = (uint32_t)va;
    pb[LAST] = (uint32_t)vb;
    return fx_read_rest<NW>(sa, tag, pa, tries, lim) && fx_read_rest<NW>(sb, tag, pb, tries, lim);
}


TG_DEV bool fx_read_unit(const uint64_t *src, uint32_t tag, uint32_t (&pay)[FX_QW], uint32_t lim) {
    return fx_read_words<FX_QW>(src, tag, pay, lim);
}

template <int UG, int UD>
__global__ __launch_bounds__(FX_THREADS) void k_experts(FxArgs A, Shape s) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int bad;
    __shared__ int sidx[MAX_K];
    __shared__ float sw[MAX_K];
    const int tid = threadIdx.x, RD = A.rd, k = s.k, nb = s.nbI, nbp = round4(nb), I = s.I, H = s.H;
    const int lrd = __builtin_ctz(RD);  // RD is a power of two
    const int ust = round4(nb) + 4;
    const uint32_t tag = __hip_atomic_load(const_cast<uint32_t *>(A.ctl) + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int r0 = blockIdx.x * RD, ng = (I / GU_ROWS) * k;
    if (tid < k) {
        const int e = A.idx[tid];
        sidx[tid] = e < 0 ? 0 : (e >= s.E ? s.E - 1 : e);
        sw[tid] = A.w[tid];
    }
    if (tid == 0) bad = 0;
    float rv = 0.0f;
    if (A.resid && tid < RD) rv = A.resid[r0 + tid];
    __syncthreads();  // sidx

    // h words of this layer: one of two buffers by tag parity, so a copy of
    // a line that an L2 still holds is at least two layers old
    uint64_t *hw = A.hw + (size_t)(tag & 1u) * ng * FX_QS;

    // 1. the first gate/up unit: loads, dots (every wave), publication
    //    (wave 0)
    FxGu<UG> g;
    const int u0 = blockIdx.x;
    if (u0 < ng) {
        fx_gu_load<UG>(A.layer_pl, s, u0, sidx, g);
        fx_gu_dots<UG>(A.xq, A.xd, A.xs, s, g, smem);
        fx_gu_publish(s, u0, tag, hw, smem, A.drop);
    }
    // 2. this block's down weights (waves 3.., item p on down thread
    //    p % FX_DT), then further gate/up units
    const size_t ntb = (size_t)H * nb;
    const int items = k * RD * nb, dt = tid - FX_PT;
    uint4 wv[UD];
    uint32_t dv[UD];
    if (dt >= 0) {  // whole waves; clamped, unbranched loads inside (as k_gateup)
#pragma unroll
        for (int u = 0; u < UD; u++) {
            const int p = min(u * FX_DT + dt, items - 1);
            const int rd = (int)fdiv((uint32_t)p, s.divI), b = p - rd * nb;
            const int jj = rd >> lrd, row = r0 + (rd - (jj << lrd));
            const uint8_t *tb = A.layer_pl + (size_t)sidx[jj] * s.EB + 2 * s.GB;
            const size_t o = (size_t)row * nb + b;
            wv[u] = reinterpret_cast<const uint4 *>(tb)[o];
            dv[u] = reinterpret_cast<const uint16_t *>(tb + ntb * 16)[o];
        }
    }
    // keep these loads here, in flight during the rest (the compiler would
    // otherwise sink them next to their use)
    __asm__ volatile("" ::: "memory");
    for (int unit = u0 + gridDim.x; unit < ng; unit += gridDim.x) {
        fx_gu_load<UG>(A.layer_pl, s, unit, sidx, g);
        __syncthreads();  // wave 0 has read the previous unit's LDS
        fx_gu_dots<UG>(A.xq, A.xd, A.xs, s, g, smem);
        fx_gu_publish(s, unit, tag, hw, smem, A.drop);
    }

    // 3. waves 0..2 read h of every unit into LDS; then the down rows
    int8_t *hq = reinterpret_cast<int8_t *>(smem + fx_down_off(s));
    float *hd = reinterpret_cast<float *>(hq + (size_t)k * I);
    int *hs = reinterpret_cast<int *>(hd + k * nbp);
    float *U = reinterpret_cast<float *>(hs + k * nbp);
    float *D = U + k * RD * ust;
    if (tid < FX_PT) {
        for (int unit = tid; unit < ng; unit += FX_PT) {
            uint32_t pay[FX_QW];
            const bool ok = fx_read_unit(hw + (size_t)unit * FX_QS, tag, pay, A.spin);
            const int jj = unit / nb, b = unit - jj * nb;
            uint32_t *dq = reinterpret_cast<uint32_t *>(hq + (size_t)jj * I + b * QK);
#pragma unroll
            for (int wd = 0; wd < 8; wd++) dq[wd] = pay[wd];
            hd[jj * nbp + b] = __uint_as_float(pay[8]);
            hs[jj * nbp + b] = (int)pay[9];
            if (!ok) bad = 1;
        }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < UD; u++) {
        const int p = u * FX_DT + dt;
        if (dt >= 0 && p < items) {
            const int rd = (int)fdiv((uint32_t)p, s.divI), b = p - rd * nb;
            const int jj = rd >> lrd;
            const int S = dot_q4_q8(wv[u], reinterpret_cast<const int *>(hq + (size_t)jj * I + b * QK)) -
                          8 * hs[jj * nbp + b];
            U[rd * ust + b] = (float)S * h2f(dv[u]);
        }
    }
    __syncthreads();
    if (tid < k * RD) D[tid] = chain4(U + tid * ust, hd + (tid >> lrd) * nbp, nb);
    __syncthreads();
    if (tid < RD) {
        const float acc = combine_slots(sw, D, RD, k, tid);
        float o = A.resid ? rv + acc : acc;
        if (bad) o = __builtin_nanf("");
        A.out[r0 + tid] = o;
    }
    if (tid == 0 && bad) __hip_atomic_store(A.err, 3u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ============================================================ one-token layer, routing inside
// One launch per layer that also routes: the layer before it (or the
// prologue k_dec_part, for the first layer of a call) leaves, per group g of
// RG output rows, the router's partial sums of that group for this layer's
// router, part[e][g] = fma chain over the group of W[e][i] * x[i] and
// part[E][g] = fma chain of x[i]^2 (the chains k_route_dec forms).  The grid
// has one block per chunk of `rd` output rows (rd = 8, 16 or 32; GQ = 32 / rd
// chunks per group, the blocks of a group on one XCD).  Every block
//   1. adds the G partials of each expert, and of the squares, in ascending
//      group order (the order of k_route_dec), scales by the RMS factor,
//      ranks, and forms the renormalised top-k weights: the same values in
//      every block, from the same inputs by the same steps;
//   2. forms Q8_0(x * s) in its LDS and runs its gate/up units as k_experts
//      (units go to the blocks that do not own a group first), publishing h
//      as tagged words;
//   3. loads its down rows for the k experts (all threads, issued before it
//      waits), reads every h word, dots, chains, combines and adds the
//      residual (as k_experts);
// and then, per group, the blocks other than the group's owner (its last
// chunk) publish their combined rows as tagged words, and the owner, with
// all RG rows, forms the next layer's partials of the group.  Waits: h (all
// blocks) and the group's rows (owners); every block publishes what it owes
// before it waits, so no wait depends on a block that is not running.
// Tags: the prologue advances the generation word past every layer of the
// call; a layer `back` launches before the call's last takes the
// generation `back` steps before it.  Polls are bounded; when one runs out
// the block sets *err and writes NaN rows (and NaN partials).
constexpr int LD_PC = 16;  // float4 of partials per load round of one thread
constexpr int LD_EMAX = 128;  // experts per layer of the routed launch (keys padded to this)

struct LdArgs {
    const uint8_t *layer_pl;
    const float *x;         // this layer's input row (H)
    const float *gn;        // this layer's FFN norm weight (H)
    const float *part_in;   // [E + 1][G] partials of x for this layer's router
    const float *wr_next;   // next layer's router [E][H], or null (no partials out)
    float *part_out;        // [E + 1][G] partials of out for the next layer
    uint64_t *hw;           // [2][k * I/32][FX_QS] tagged h blocks, by tag parity
    uint64_t *ow;           // [2][H] tagged combined rows of the group hand-off, by tag parity
    const uint32_t *ctl;    // ctl[1]: generation of the call's last layer
    uint32_t back;          // launches of this call after this one
    uint32_t *err;
    const float *resid;
    float *out;
    int32_t *idx;           // this layer's top-k ids and weights (block 0 writes them)
    float *w;
    float eps;
    int rd;                 // output rows per block (grid = H / rd)
    uint32_t spin;          // poll bound (fault_spin_limit())
    int drop;               // h line (unit, or half unit) left unpublished (-1 in normal use)
};

// generation `back` steps before g in next_gen's cycle 1 .. 2^31 - 1
TG_DEV uint32_t gen_back(uint32_t g, uint32_t back) {
    const int64_t M = 0x7FFFFFFF;
    int64_t v = ((int64_t)(g == 0u ? 1u : g) - 1 - (int64_t)back) % M;
    if (v < 0) v += M;
    return (uint32_t)(v + 1);
}

// Block b's chunk and role.  With NB % (8 GQ) == 0 the GQ chunks of group g
// go to blocks that share b % 8 (one XCD when blocks are dealt round robin
// over 8 XCDs); `rank` orders blocks for the gate/up units, non-owners
// first.
struct LdRole {
    int chunk, group, q, rank;
    bool owner;
};

TG_DEV LdRole ld_role(int b, int NB, int GQ) {
    LdRole r;
    if (NB % (8 * GQ) == 0) {
        const int x = b % 8, q = (b / 8) % GQ, t = b / (8 * GQ);
        r.group = t * 8 + x;
        r.q = q;
    } else {
        r.group = b / GQ;
        r.q = b % GQ;
    }
    r.chunk = r.group * GQ + r.q;
    r.owner = r.q == GQ - 1;
    const int n_groups = NB / GQ;
    r.rank = r.owner ? n_groups * (GQ - 1) + r.group : r.group * (GQ - 1) + r.q;
    return r;
}

// LDS: the gate/up part, then the down part (k_experts' layout for rd rows),
// the group's RG combined rows and the next router's columns [E][RG + 1] ...
// ... and one arrival flag per gate/up unit (nonzero once that unit's h
// block is in LDS).
__host__ __device__ inline size_t ld_lds_bytes(const Shape &s, int rd) {
    return fx_down_off(s) + fx_down_lds_bytes(s.k, s.I, s.nbI, rd) + 4 * (size_t)RG + 4 * (size_t)s.E * (RG + 1) +
           4 * (size_t)s.k * s.nbI;
}

// Index maps of one thread's weight items, formed at launch (they do not
// depend on the routing), so the phases after the routing only add the
// selected expert's base and read LDS at precomputed offsets.  Gate/up
// unit (m, j): item u is p = u * FX_THREADS + tid (clamped) of the unit's
// 2 * GU_ROWS * nbH blocks, row rd = p >> lnbH (gate rows 0..31, up rows
// 32..63), column block cb = p & (nbH - 1).
template <int UG>
struct LdGu {
    uint32_t off[UG];  // byte offset of the nibbles inside the expert
    uint32_t soff[UG]; // byte offset of the scale
    uint32_t pk[UG];   // U index << 8 | cb
};

template <int UG>
TG_DEV void ld_gu_map(const Shape &s, int m, int lnbh, int usth, LdGu<UG> &M) {
    constexpr int RT = GU_ROWS;
    const int nbh = s.nbH, items = 2 * RT * nbh, tid = threadIdx.x;
    const uint32_t ntb = (uint32_t)s.I * nbh;
#pragma unroll
    for (int u = 0; u < UG; u++) {
        const int p = min(u * FX_THREADS + tid, items - 1);
        const int rd = p >> lnbh, cb = p & (nbh - 1);
        const int mat = rd >= RT ? 1 : 0;
        const uint32_t idx = (uint32_t)((m * RT + rd - mat * RT) * nbh + cb);
        const uint32_t tb = mat ? (uint32_t)s.GB : 0u;
        M.off[u] = tb + 16u * idx;
        M.soff[u] = tb + 16u * ntb + 2u * idx;
        M.pk[u] = ((uint32_t)(rd * usth + cb) << 8) | (uint32_t)cb;
    }
}

template <int UG>
TG_DEV void ld_gu_load(const uint8_t *ex, const LdGu<UG> &M, FxGu<UG> &g) {
#pragma unroll
    for (int u = 0; u < UG; u++) {
        g.wv[u] = *reinterpret_cast<const uint4 *>(ex + M.off[u]);
        g.dv[u] = *reinterpret_cast<const uint16_t *>(ex + M.soff[u]);
    }
}

// The unit's block dots into U (LDS), at the precomputed offsets.
template <int UG>
TG_DEV void ld_gu_dots(const Shape &s, const LdGu<UG> &M, const FxGu<UG> &g, uint8_t *smem, int rows = GU_ROWS) {
    const int nbh = s.nbH, H = s.H, items = 2 * rows * nbh, tid = threadIdx.x;
    const int8_t *xq = reinterpret_cast<const int8_t *>(smem);
    const int *xs = reinterpret_cast<const int *>(xq + H + 4 * round4(nbh));
    float *U = reinterpret_cast<float *>(smem + H + 8 * round4(nbh));
    lds_barrier();  // Q8_0 x in LDS; the previous unit's U read
    if (items >= UG * FX_THREADS) {  // uniform: every item exists, so no branch per item (30B: +0.8%)
#pragma unroll
        for (int u = 0; u < UG; u++) {
            const int cb = (int)(M.pk[u] & 255u), ui = (int)(M.pk[u] >> 8);
            const int S = dot_q4_q8(g.wv[u], reinterpret_cast<const int *>(xq + cb * QK)) - 8 * xs[cb];
            U[ui] = (float)S * h2f((uint16_t)at_use(g.dv[u]));
        }
    } else {
#pragma unroll
        for (int u = 0; u < UG; u++) {
            if (u * FX_THREADS + tid < items) {
                const int cb = (int)(M.pk[u] & 255u), ui = (int)(M.pk[u] >> 8);
                const int S = dot_q4_q8(g.wv[u], reinterpret_cast<const int *>(xq + cb * QK)) - 8 * xs[cb];
                U[ui] = (float)S * h2f((uint16_t)at_use(g.dv[u]));
            }
        }
    }
    lds_barrier();
}

// The leading arguments (the partials' address, E, G) arrive preloaded in
// SGPRs (this file is built with kernarg preloading), so the first round of
// partial loads is issued before any argument is read from memory.
// Half units (the layer launch when a shape has more units than blocks):
// half unit hu = 2 u + side takes rows [16 side, 16 side + 16) of unit u's
// gate and of its up rows, so the 32 h values of a unit come from two
// blocks and every block carries the same number of half units.  Item u of a
// thread: p = u * FX_THREADS + tid of the half unit's 2 * 16 * nbH blocks, row
// rd = p >> lnbH (gate 0..15, up 16..31), dotted into U row ubase + rd.
constexpr int HU_ROWS = GU_ROWS / 2;
constexpr int HU_QS = 16;  // tagged words per half unit: its 16 h values, one 128-byte line

template <int UG>
TG_DEV void ld_hu_map(const Shape &s, int m, int side, int ubase, int lnbh, int usth, LdGu<UG> &M) {
    const int nbh = s.nbH, items = 2 * HU_ROWS * nbh, tid = threadIdx.x;
    const uint32_t ntb = (uint32_t)s.I * nbh;
#pragma unroll
    for (int u = 0; u < UG; u++) {
        const int p = min(u * FX_THREADS + tid, items - 1);
        const int rd = p >> lnbh, cb = p & (nbh - 1);
        const int mat = rd >= HU_ROWS ? 1 : 0;
        const uint32_t idx = (uint32_t)((m * GU_ROWS + side * HU_ROWS + rd - mat * HU_ROWS) * nbh + cb);
        const uint32_t tb = mat ? (uint32_t)s.GB : 0u;
        M.off[u] = tb + 16u * idx;
        M.soff[u] = tb + 16u * ntb + 2u * idx;
        M.pk[u] = ((uint32_t)((ubase + rd) * usth + cb) << 8) | (uint32_t)cb;
    }
}

// The block's last wave: the chains of U rows 0..63 (half unit huA in rows
// 0..31, huB, if >= 0, in rows 32..63), SwiGLU of each half's 16 rows, and
// the 16 h values of each half published as tagged words (lanes 0..15: huA,
// 32..47: huB).  Readers form the Q8_0 block of a unit from its two halves.
TG_DEV void fx_hu_publish(const Shape &s, int huA, int huB, uint32_t tag, uint64_t *hw, const uint8_t *smem,
                          int drop) {
    const int nb = s.nbH, ust = round4(nb) + 4, H = s.H, tid = threadIdx.x;
    const float *xd = reinterpret_cast<const float *>(smem + H);
    const float *U = xd + 2 * round4(nb);
    if (tid >= FX_THREADS - WAVE) {  // the last wave: wave 0 polls first and should not wait for these stores
        const int ln = tid - (FX_THREADS - WAVE);
        const float a = chain4(U + ln * ust, xd, nb);
        const float gv = __shfl(a, ln, WAVE), uv = __shfl(a, (ln + HU_ROWS) & (WAVE - 1), WAVE);
        const int l = ln & 31, half = ln >> 5;
        const int hu = half ? huB : huA;
        if (l < HU_ROWS && hu >= 0 && hu != drop)
            ll_put(hw + (size_t)hu * HU_QS + l, __float_as_uint(silu_mul(gv, uv)), tag);
    }
}

// Q8_0 of a unit's 32 h values in one thread, the steps of q8_lane (the same
// bits for finite values: the maximum of |v| does not depend on the order it
// is taken in): the packed bytes, the scale as float(half(d)), the sum.
TG_DEV void q8_block32(const float (&v)[32], uint32_t (&wq)[8], float &dscale, int &qsum) {
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const float o = fabsf(v[i]);
        a = o > a ? o : a;
    }
    const float d = a / 127.0f;
    const float inv = a > 0.0f ? 127.0f / a : 0.0f;
    int sum = 0;
#pragma unroll
    for (int w = 0; w < 8; w++) {
        uint32_t word = 0u;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int q = (int)__builtin_rintf(v[4 * w + b] * inv);
            sum += q;
            word |= (uint32_t)(q & 255) << (8 * b);
        }
        wq[w] = word;
    }
    dscale = h2f(f2h(d));
    qsum = sum;
}

template <int UG, int UD, bool HU, bool XS>
__global__ __launch_bounds__(FX_THREADS) void k_layer_dec(const float *__restrict__ part_in, int pe, int pg, LdArgs A,
                                                          Shape s) {
    float4 pv0[LD_PC];
    if ((int)threadIdx.x <= pe) {
        const float4 *row = reinterpret_cast<const float4 *>(part_in + (size_t)threadIdx.x * pg);
#pragma unroll
        for (int q = 0; q < LD_PC; q++) pv0[q] = row[min(q, pg / 4 - 1)];
    }
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ __align__(16) uint64_t keys[LD_EMAX];
    __shared__ int rcnt[LD_EMAX];
    __shared__ float slog[LD_EMAX];
    __shared__ int sidx[MAX_K];
    __shared__ float sw[MAX_K];
    __shared__ float ssc;
    __shared__ int bad;
    const int tid = threadIdx.x, k = s.k, E = s.E, H = s.H, I = s.I, G = H / RG, RD = A.rd, GQ = RG / RD;
    const int lrd = __builtin_ctz(RD);  // RD is a power of two
    const int nb = s.nbI, nbp = round4(nb), ust = round4(nb) + 4;
    const int lnbh = __builtin_ctz(s.nbH), usth = round4(s.nbH) + 4;  // nbH is a power of two
    const int ng = (I / GU_ROWS) * k, NB = gridDim.x, mI = I / GU_ROWS;
    const int nu = HU ? 2 * ng : ng;  // work units: units, or half units
    const LdRole role = ld_role(blockIdx.x, NB, GQ);
    // expert-sliced down (XS): block b dots slot jx = b % k over the rows
    // [r0, r0 + k RD) (so it reads the h of one expert only) and publishes
    // them; each group's owner combines the k slots of its RG rows.
    // Otherwise block b takes its RD rows of every slot.
    const int jx = XS ? (int)blockIdx.x % k : 0;
    const int r0 = XS ? ((int)blockIdx.x / k) * (k * RD) : role.chunk * RD;
    const int g0 = role.group * RG;
    const uint32_t tag =
        gen_back(__hip_atomic_load(const_cast<uint32_t *>(A.ctl) + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                 A.back);
    uint64_t *hw = A.hw + (size_t)(tag & 1u) * ng * (HU ? 2 * HU_QS : FX_QS);
    uint64_t *ow = A.ow + (size_t)(tag & 1u) * (XS ? (size_t)k * H : (size_t)H);
    const bool nx = role.owner && A.wr_next;

    // 0. loads that depend on nothing: x and the norm weight (the threads
    //    that quantize it, waves 1..), the residual rows, (owners) the next
    //    router's columns of the group, then the partials
    float4 xa = make_float4(0.f, 0.f, 0.f, 0.f), xb = xa, ga = xa, gb = xa;
    const int u0 = role.rank;  // first gate/up unit (half unit)
    const int qt = tid - WAVE;
    const bool qon = u0 < nu && qt >= 0 && qt < H / 8;
    if (qon) {
        xa = reinterpret_cast<const float4 *>(A.x)[2 * qt];
        xb = reinterpret_cast<const float4 *>(A.x)[2 * qt + 1];
        ga = reinterpret_cast<const float4 *>(A.gn)[2 * qt];
        gb = reinterpret_cast<const float4 *>(A.gn)[2 * qt + 1];
    }
    // deep unit loads (UG > 4): the unit map is formed after the routing and
    // the down map after the units (the maps and the loads they address
    // never hold registers at once), and the residual rows and the down
    // scales go to LDS without registers (dsl: [UD][FX_THREADS] scale words,
    // then the residual rows), since a loaded value the compiler spills is
    // waited for on the spot
    constexpr bool DOWN_FIRST = UG <= 4;
    const int dsl_off = (int)ld_lds_bytes(s, RD);
    const uint32_t *dsl = reinterpret_cast<const uint32_t *>(smem + dsl_off);
    float rv = 0.0f;
    // the residual rows this block combines: its RD rows, or (XS) its group's
    // RG rows when it owns the group
    const int rrow = XS ? g0 : r0, rn = XS ? RG : RD;
    const bool rown = !XS || role.owner;
    if constexpr (DOWN_FIRST) {
        if (A.resid && rown && tid < rn) rv = A.resid[rrow + tid];
    } else {
        if (A.resid && rown && tid < WAVE)  // wave 0; the wait before the unit loads retires it
            lds_dma4(A.resid + rrow + min(tid, rn - 1), lds_addr(smem, dsl_off + 4 * UD * FX_THREADS));
    }
    float4 wn = make_float4(0.f, 0.f, 0.f, 0.f);
    if (nx && tid < E * (RG / 4))
        wn = reinterpret_cast<const float4 *>(A.wr_next + (size_t)(tid >> 3) * H + (size_t)role.group * RG)[tid & 7];
    if (tid == 0) bad = 0;
    // arrival flags of the h blocks (LDS starts undefined): cleared before
    // the first barrier, set by the polling waves, read by the down dots
    int *uflag = reinterpret_cast<int *>(smem + ld_lds_bytes(s, RD) - 4 * (size_t)ng);
    for (int i = tid; i < ng; i += FX_THREADS) uflag[i] = 0;

    // 1. routing: thread e <= E adds row e of the partials in ascending group
    //    order (LD_PC float4 loaded per round, all before the adds)
    if (tid <= E) {
        const float4 *row = reinterpret_cast<const float4 *>(part_in + (size_t)tid * G);
        float tot = 0.0f;
        for (int c = 0; c < G / 4; c += LD_PC) {
            float4 pv[LD_PC];
#pragma unroll
            for (int q = 0; q < LD_PC; q++) pv[q] = c == 0 ? pv0[q] : row[min(c + q, G / 4 - 1)];
#pragma unroll
            for (int q = 0; q < LD_PC; q++)
                if (c + q < G / 4) {
                    tot = tot + pv[q].x; tot = tot + pv[q].y; tot = tot + pv[q].z; tot = tot + pv[q].w;
                }
        }
        if (tid < E)
            slog[tid] = tot;
        else
            ssc = rms_scale(tot, H, A.eps);
    }
    // while the partials load: the index maps of this thread's weight items
    LdGu<UG> gm;
    if (DOWN_FIRST) ld_gu_map<UG>(s, u0 % mI, lnbh, usth, gm);
    // down item u: byte offset of its row block; (slot * RD + row) << 16 | block.
    // Every thread takes down items, the polling waves included: their polls
    // then start when their down loads have landed (vmcnt retires in order),
    // which keeps the poll traffic off the fabric while the down stream is
    // in flight (measured faster than keeping the polling waves free).
    const int items = k * RD * nb;
    const int dthr = FX_THREADS, dt = tid;  // every thread; the polls wait for these loads, which thins them
    // item u of this thread: (slot * RD + row) or (XS) the slice row, and the
    // block; derived where used, so no register holds the map while the
    // loads are in flight
    auto dpos = [&](int u, int &rdi, int &b) {
        const int p = min(u * dthr + max(dt, 0), items - 1);
        rdi = (int)fdiv((uint32_t)p, s.divI);
        b = p - rdi * nb;
    };
    auto doff_of = [&](int rdi, int b) -> uint32_t {
        const int row = XS ? r0 + rdi : r0 + (rdi & (RD - 1));
        return (uint32_t)(2 * s.GB) + 16u * (uint32_t)(row * nb + b);
    };
    __syncthreads();
    const float sc = ssc;
    // keys (the experts beyond E rank below every logit)
    if (tid < LD_EMAX) {
        uint64_t key = 0;
        if (tid < E) {
            const float l = slog[tid] * sc;
            slog[tid] = l;
            key = rank_key(l, tid);
        }
        keys[tid] = key;
        rcnt[tid] = 0;
    }
    lds_barrier();
    // rank = number of larger keys: thread (e, part) = (tid % 128, tid / 128)
    // counts among keys [16 part, 16 part + 16), LDS broadcasts
    {
        const int e = tid & (LD_EMAX - 1), part = tid >> 7;
        const uint64_t my = keys[e];
        const ulonglong2 *kp = reinterpret_cast<const ulonglong2 *>(keys + 16 * part);
        ulonglong2 kk[8];
#pragma unroll
        for (int q = 0; q < 8; q++) kk[q] = kp[q];
        int cnt = 0;
#pragma unroll
        for (int q = 0; q < 8; q++) cnt += (kk[q].x > my ? 1 : 0) + (kk[q].y > my ? 1 : 0);
        if (e < E && cnt) atomicAdd(rcnt + e, cnt);
    }
    lds_barrier();
    if (tid < E && rcnt[tid] < k) sidx[rcnt[tid]] = tid;
    // the first unit's weights are in flight while wave 0 forms the softmax
    // and waves 1.. Q8_0((x * s) * g) into the gate/up LDS layout; the
    // normed x is formed (and pinned) before the unit loads are issued, so
    // the Q8_0 waits for no load
    float xsv[8];
    if (qon) {
        const float v[8] = {(xa.x * sc) * ga.x, (xa.y * sc) * ga.y, (xa.z * sc) * ga.z, (xa.w * sc) * ga.w,
                            (xb.x * sc) * gb.x, (xb.y * sc) * gb.y, (xb.z * sc) * gb.z, (xb.w * sc) * gb.w};
#pragma unroll
        for (int c = 0; c < 8; c++) xsv[c] = __uint_as_float(at_use(__float_as_uint(v[c])));
    }
    // the loads issued at launch (x, the residual rows, the router columns)
    // landed long ago: an explicit wait for them here leaves the unit's
    // loads as the only ones in flight, so nothing below waits for those
    __builtin_amdgcn_s_waitcnt(VMCNT0);
    lds_barrier();  // sidx
    // this block's down weights: issued after the first unit's publication
    // with shallow unit loads (UG <= 4; issued with the unit's loads they
    // slow the unit's stream by as much as they add), after the units with
    // deep ones
    const size_t ntb = (size_t)H * nb;
    uint4 wv[UD];
    uint32_t dv[UD];
    auto down_loads = [&]() {
        if (dt >= 0) {  // whole waves; clamped, unbranched loads inside
            if constexpr (DOWN_FIRST) {
#pragma unroll
                for (int u = 0; u < UD; u++) {
                    int rdi, b;
                    dpos(u, rdi, b);
                    const uint32_t doff = doff_of(rdi, b);
                    const uint8_t *ex = A.layer_pl + (size_t)sidx[XS ? jx : rdi >> lrd] * s.EB;
                    wv[u] = *reinterpret_cast<const uint4 *>(ex + doff);
                    const uint32_t bi = (doff - (uint32_t)(2 * s.GB)) >> 4;
                    dv[u] = reinterpret_cast<const uint16_t *>(ex + 2 * s.GB + ntb * 16)[bi];
                }
            } else {
                // the scales first (the word holding each: nb is even, so
                // block b's scale is its high half when b is odd), then the
                // nibbles: a wait for any nibble load covers every scale
#pragma unroll
                for (int u = 0; u < UD; u++) {
                    int rdi, b;
                    dpos(u, rdi, b);
                    const uint8_t *ex = A.layer_pl + (size_t)sidx[XS ? jx : rdi >> lrd] * s.EB;
                    const uint32_t bi = (doff_of(rdi, b) - (uint32_t)(2 * s.GB)) >> 4;
                    lds_dma4(ex + 2 * s.GB + ntb * 16 + (size_t)(bi & ~1u) * 2,
                             lds_addr(smem, dsl_off + 4 * (u * FX_THREADS + (tid & ~(WAVE - 1)))));
                }
#pragma unroll
                for (int u = 0; u < UD; u++) {
                    int rdi, b;
                    dpos(u, rdi, b);
                    const uint8_t *ex = A.layer_pl + (size_t)sidx[XS ? jx : rdi >> lrd] * s.EB;
                    wv[u] = *reinterpret_cast<const uint4 *>(ex + doff_of(rdi, b));
                }
            }
        }
        __asm__ volatile("" ::: "memory");  // keep the down loads in flight from here
    };
    FxGu<UG> g;
    // (half units) the first two: hu0 = u0 into U rows 0..31, hu1 = u0 + NB
    // into rows 32..63, their loads in flight together
    constexpr int UH = UG / 2 > 0 ? UG / 2 : 1;
    LdGu<UH> hma, hmb;
    FxGu<UH> hga, hgb;
    const int hu1 = u0 + NB;
    // (half units) odd blocks stream one half unit first and then two, even
    // blocks two and then one: the loads of one set run while the other
    // dots, so the fabric is not left idle while every block dots at once
    // (with one order for all blocks the 235B launch took 1.5 us longer)
    const bool one_first = HU && (blockIdx.x & 1) && u0 + 2 * NB < nu;
    if constexpr (HU) {
        if (u0 < nu) {  // nested like the dots below, so no path leaves a load unconsumed
            const int un = u0 >> 1;
            ld_hu_map<UH>(s, un % mI, u0 & 1, 0, lnbh, usth, hma);
            ld_gu_load<UH>(A.layer_pl + (size_t)sidx[un / mI] * s.EB, hma, hga);
            if (hu1 < nu && !one_first) {
                const int un1 = hu1 >> 1;
                ld_hu_map<UH>(s, un1 % mI, hu1 & 1, GU_ROWS, lnbh, usth, hmb);
                ld_gu_load<UH>(A.layer_pl + (size_t)sidx[un1 / mI] * s.EB, hmb, hgb);
            }
        }
    } else {
        if (!DOWN_FIRST) ld_gu_map<UG>(s, u0 % mI, lnbh, usth, gm);
        if (u0 < ng) ld_gu_load<UG>(A.layer_pl + (size_t)sidx[u0 / mI] * s.EB, gm, g);
    }
    if (tid < WAVE) {
        const float wj = topk_softmax_lane(slog, sidx, k);
        if (tid < k) {
            const int j = k - 1 - tid;
            sw[j] = wj;
            if (blockIdx.x == 0) {
                A.idx[j] = sidx[j];
                A.w[j] = wj;
            }
        }
    }
    int8_t *xq = reinterpret_cast<int8_t *>(smem);
    float *xd = reinterpret_cast<float *>(xq + H);
    int *xs = reinterpret_cast<int *>(xd + round4(s.nbH));
    if (qon) q8_group8(xsv, true, qt * 8, xq, xd, xs);

    if constexpr (HU) {
        if (one_first) {  // uniform: u0, then u0 + NB and u0 + 2 NB together
            ld_gu_dots<UH>(s, hma, hga, smem, HU_ROWS);
            fx_consume<UH>(hga);
            fx_hu_publish(s, u0, -1, tag, hw, smem, A.drop);
            const int hb = u0 + NB, hc = u0 + 2 * NB;
            const int ub = hb >> 1, uc = hc >> 1;
            ld_hu_map<UH>(s, ub % mI, hb & 1, 0, lnbh, usth, hma);
            ld_gu_load<UH>(A.layer_pl + (size_t)sidx[ub / mI] * s.EB, hma, hga);
            ld_hu_map<UH>(s, uc % mI, hc & 1, GU_ROWS, lnbh, usth, hmb);
            ld_gu_load<UH>(A.layer_pl + (size_t)sidx[uc / mI] * s.EB, hmb, hgb);
            ld_gu_dots<UH>(s, hma, hga, smem, HU_ROWS);
            fx_consume<UH>(hga);
            ld_gu_dots<UH>(s, hmb, hgb, smem, HU_ROWS);
            fx_consume<UH>(hgb);
            fx_hu_publish(s, hb, hc, tag, hw, smem, A.drop);
        } else if (u0 < nu) {  // uniform
            ld_gu_dots<UH>(s, hma, hga, smem, HU_ROWS);
            fx_consume<UH>(hga);
            if (hu1 < nu) {
                ld_gu_dots<UH>(s, hmb, hgb, smem, HU_ROWS);
                fx_consume<UH>(hgb);
            }
            fx_hu_publish(s, u0, hu1 < nu ? hu1 : -1, tag, hw, smem, A.drop);
        }
        // 2. further half units, one at a time
        for (int hu = u0 + (one_first ? 3 : 2) * NB; hu < nu; hu += NB) {
            LdGu<UH> hm2;
            const int un = hu >> 1;
            ld_hu_map<UH>(s, un % mI, hu & 1, 0, lnbh, usth, hm2);
            ld_gu_load<UH>(A.layer_pl + (size_t)sidx[un / mI] * s.EB, hm2, hga);
            ld_gu_dots<UH>(s, hm2, hga, smem, HU_ROWS);
            fx_consume<UH>(hga);
            fx_hu_publish(s, hu, -1, tag, hw, smem, A.drop);
        }
    } else {
        if (u0 < ng) {
            ld_gu_dots<UG>(s, gm, g, smem);
            fx_gu_publish(s, u0, tag, hw, smem, A.drop);
        }
        if (DOWN_FIRST) down_loads();
        // 2. further gate/up units
        for (int unit = u0 + NB; unit < ng; unit += NB) {
            LdGu<UG> gm2;
            ld_gu_map<UG>(s, unit % mI, lnbh, usth, gm2);
            ld_gu_load<UG>(A.layer_pl + (size_t)sidx[unit / mI] * s.EB, gm2, g);
            ld_gu_dots<UG>(s, gm2, g, smem);
            fx_gu_publish(s, unit, tag, hw, smem, A.drop);
        }
    }
    if (!DOWN_FIRST) down_loads();

    // 3. waves 0..2 read h of every unit into LDS (after the gate/up part,
    //    which wave 0 may still be reading); then the down rows
    int8_t *hq = reinterpret_cast<int8_t *>(smem + fx_down_off(s));
    float *hd = reinterpret_cast<float *>(hq + (size_t)k * I);
    int *hs = reinterpret_cast<int *>(hd + k * nbp);
    float *U = reinterpret_cast<float *>(hs + k * nbp);
    float *D = U + k * RD * ust;
    float *xo = D + k * RD;
    float *wl = xo + RG;  // [E][RG + 1]
    // (half units: a unit's two lines are polled together; more polling
    // waves were slower, the coherent poll traffic grows with them)
    if (tid < FX_PT) {
        const int nun = XS ? nb : ng;  // the units to read: slot jx's, or every unit
        for (int uu = tid; uu < nun; uu += FX_PT) {
            const int unit = XS ? jx * nb + uu : uu;
            uint32_t pay[FX_QW];
            bool ok;
            if constexpr (HU) {  // the unit's two halves, then its Q8_0 block here
                uint32_t pa[HU_QS], pb[HU_QS];
                ok = fx_read_pair<HU_QS>(hw + (size_t)(2 * unit) * HU_QS, hw + (size_t)(2 * unit + 1) * HU_QS, tag,
                                         pa, pb, A.spin);
                float v[2 * HU_QS];
#pragma unroll
                for (int i = 0; i < HU_QS; i++) {
                    v[i] = __uint_as_float(pa[i]);
                    v[HU_QS + i] = __uint_as_float(pb[i]);
                }
                uint32_t wq[8];
                float dsc;
                int qs;
                q8_block32(v, wq, dsc, qs);
#pragma unroll
                for (int wd = 0; wd < 8; wd++) pay[wd] = wq[wd];
                pay[8] = __float_as_uint(dsc);
                pay[9] = (uint32_t)qs;
            } else {
                ok = fx_read_unit(hw + (size_t)unit * FX_QS, tag, pay, A.spin);
            }
            const int jj = XS ? 0 : unit / nb, b = unit - (XS ? jx : jj) * nb;
            uint32_t *dq = reinterpret_cast<uint32_t *>(hq + (size_t)jj * I + b * QK);
#pragma unroll
            for (int wd = 0; wd < 8; wd++) dq[wd] = pay[wd];
            hd[jj * nbp + b] = __uint_as_float(pay[8]);
            hs[jj * nbp + b] = (int)pay[9];
            if (!ok) bad = 1;
            // release: the copies above are in LDS before the flag is
            __hip_atomic_store(uflag + uu, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }
    if (nx && tid < E * (RG / 4)) {
        const int e = tid >> 3, c = 4 * (tid & 7);
        wl[e * (RG + 1) + c] = wn.x;
        wl[e * (RG + 1) + c + 1] = wn.y;
        wl[e * (RG + 1) + c + 2] = wn.z;
        wl[e * (RG + 1) + c + 3] = wn.w;
    }
    // each down dot starts once its unit's h block is in LDS, so the dots run
    // while later units are still on their way.  The polling waves finish
    // every poll of theirs (bounded) before their own dots, so each flag is
    // set; the wait here is bounded too.  (Deep unit loads: at most the UD
    // nibble loads still in flight, so the older scale loads have landed;
    // the flag's acquire keeps the scale reads after this wait.)
    if constexpr (!DOWN_FIRST) __builtin_amdgcn_s_waitcnt(VMCNT0 | UD);
#pragma unroll
    for (int u = 0; u < UD; u++) {
        if (dt >= 0 && u * dthr + dt < items) {
            int rdi, b;
            dpos(u, rdi, b);
            const int jj = XS ? 0 : rdi >> lrd;
            const int unit = (int)__umul24((uint32_t)jj, (uint32_t)nb) + b;
            uint32_t tries = 0;
            while (__hip_atomic_load(uflag + unit, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == 0) {
                if (++tries >= A.spin) {
                    bad = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            const int4 *h4 = reinterpret_cast<const int4 *>(hq + __umul24((uint32_t)jj, (uint32_t)I) + b * QK);
            const int4 ha = h4[0], hb = h4[1];
            const int hx[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
            const int S = dot_q4_q8(wv[u], hx) - 8 * hs[(int)__umul24((uint32_t)jj, (uint32_t)nbp) + b];
            uint32_t sv;
            if constexpr (DOWN_FIRST)
                sv = at_use(dv[u]);
            else
                sv = dsl[u * FX_THREADS + tid] >> (16 * (b & 1));
            U[(int)__umul24((uint32_t)rdi, (uint32_t)ust) + b] = (float)S * h2f((uint16_t)sv);
        }
    }
    lds_barrier();
    if constexpr (XS) {
        // the chains of the slice's k RD rows of slot jx, published for the
        // owners of their groups
        if (tid < k * RD) {
            float dvl = chain4(U + tid * ust, hd, nb);
            if (bad) dvl = __builtin_nanf("");
            ll_put(ow + (size_t)jx * H + r0 + tid, __float_as_uint(dvl), tag);
        }
        if (!role.owner) {  // uniform
            if (tid == 0 && bad) __hip_atomic_store(A.err, 3u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
        // (owners) the k slots of the group's RG rows (over the unused
        // slots of hq), combined in the reference's order, plus the
        // residual
        float *dsum = reinterpret_cast<float *>(hq + ((I + 15) & ~15));
        if (tid < k * RG) {
            const int jj = tid / RG, r = tid - jj * RG;
            const uint64_t *src = ow + (size_t)jj * H + g0 + r;
            uint64_t v = ll_get(src);
            uint32_t tries = 0;
            while ((uint32_t)(v >> 32) != tag) {
                if (++tries >= A.spin) {
                    bad = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
                v = ll_get(src);
            }
            dsum[tid] = __uint_as_float((uint32_t)v);
        }
        __syncthreads();
        if (tid < RG) {
            const float acc = combine_slots(sw, dsum, RG, k, tid);
            if constexpr (!DOWN_FIRST) rv = __uint_as_float(dsl[UD * FX_THREADS + tid]);
            float o = A.resid ? rv + acc : acc;
            if (bad) o = __builtin_nanf("");
            A.out[g0 + tid] = o;
            xo[tid] = o;
        }
        if (!nx) {  // uniform
            if (tid == 0 && bad) __hip_atomic_store(A.err, 3u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
    }
    // chains and combine: with k * RD <= 64 one wave holds every (slot, row)
    // chain and gathers a row's k slots by lane shuffles
    float o = 0.0f;
    if (XS) {
    } else if (k * RD <= WAVE) {
        if (tid < WAVE) {
            const int t = tid < k * RD ? tid : 0;
            const float dvl = chain4(U + t * ust, hd + (t >> lrd) * nbp, nb);
            const int r = tid & (RD - 1);
            // k * RD <= 64 and RD >= 8: k <= 8 slots, all shuffled ahead of
            // the chain (one LDS round trip instead of one per slot)
            float dd[8], ww[8];
#pragma unroll
            for (int c = 0; c < 8; c++) {
                dd[c] = __shfl(dvl, min(c, k - 1) * RD + r, WAVE);
                ww[c] = sw[min(c, k - 1)];
            }
            float acc = 0.0f;
#pragma unroll
            for (int c = 7; c >= 0; c--)
                if (c < k) acc = __builtin_fmaf(ww[c], dd[c], acc);
            if constexpr (!DOWN_FIRST) rv = __uint_as_float(dsl[UD * FX_THREADS + tid]);  // after the barrier above
            o = A.resid ? rv + acc : acc;
        }
    } else {
        if (tid < k * RD) D[tid] = chain4(U + tid * ust, hd + (tid >> lrd) * nbp, nb);
        lds_barrier();
        if (tid < RD) {
            const float acc = combine_slots(sw, D, RD, k, tid);
            if constexpr (!DOWN_FIRST) rv = __uint_as_float(dsl[UD * FX_THREADS + tid]);
            o = A.resid ? rv + acc : acc;
        }
    }
    // a non-owner publishes its rows to the group's owner
    if (!XS && tid < RD) {
        if (bad) o = __builtin_nanf("");
        A.out[r0 + tid] = o;
        if (A.wr_next) {
            if (role.owner)
                xo[role.q * RD + tid] = o;
            else
                ll_put(ow + r0 + tid, __float_as_uint(o), tag);
        }
    }
    if (!XS && !nx) {  // uniform
        if (tid == 0 && bad) __hip_atomic_store(A.err, 3u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    // 4. (owners) the group's other rows, then the next layer's partials of
    //    the group from its RG rows
    const int gr0 = role.group * RG;
    if (!XS && tid < RG - RD) {
        const uint64_t *src = ow + gr0 + tid;
        uint64_t v = ll_get(src);
        uint32_t tries = 0;
        while ((uint32_t)(v >> 32) != tag) {
            if (++tries >= A.spin) {
                bad = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
            v = ll_get(src);
        }
        xo[tid] = __uint_as_float((uint32_t)v);
    }
    __syncthreads();
    const int gi = role.group;
    if (tid < E) {
        float aw = 0.0f;
#pragma unroll
        for (int r = 0; r < RG; r++) aw = __builtin_fmaf(wl[tid * (RG + 1) + r], xo[r], aw);
        A.part_out[(size_t)tid * G + gi] = bad ? __builtin_nanf("") : aw;
    } else if (tid == E) {
        float aq = 0.0f;
#pragma unroll
        for (int r = 0; r < RG; r++) aq = __builtin_fmaf(xo[r], xo[r], aq);
        A.part_out[(size_t)E * G + gi] = bad ? __builtin_nanf("") : aq;
    }
    if (tid == 0 && bad) __hip_atomic_store(A.err, 3u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Prologue of a one-token call: the partials of x for the router of the
// call's first layer (block g: group g; thread e < E the chain of expert e,
// thread E the chain of squares), and block 0 advances the generation word
// by n_layers (one generation per layer launch of the call).
__global__ __launch_bounds__(256) void k_dec_part(const float *__restrict__ Wr, const float *__restrict__ x, int E,
                                                  int H, float *__restrict__ part, uint32_t *ctl, int n_layers) {
    const int g = blockIdx.x, tid = threadIdx.x, G = H / RG;
    const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)g * RG);
    float4 xv[RG / 4];
#pragma unroll
    for (int q = 0; q < RG / 4; q++) xv[q] = x4[q];
    if (tid < E) {
        const float4 *w4 = reinterpret_cast<const float4 *>(Wr + (size_t)tid * H + (size_t)g * RG);
        float4 wv[RG / 4];
#pragma unroll
        for (int q = 0; q < RG / 4; q++) wv[q] = w4[q];
        float aw = 0.0f;
#pragma unroll
        for (int q = 0; q < RG / 4; q++) {
            aw = __builtin_fmaf(wv[q].x, xv[q].x, aw);
            aw = __builtin_fmaf(wv[q].y, xv[q].y, aw);
            aw = __builtin_fmaf(wv[q].z, xv[q].z, aw);
            aw = __builtin_fmaf(wv[q].w, xv[q].w, aw);
        }
        part[(size_t)tid * G + g] = aw;
    } else if (tid == E) {
        float aq = 0.0f;
#pragma unroll
        for (int q = 0; q < RG / 4; q++) {
            aq = __builtin_fmaf(xv[q].x, xv[q].x, aq);
            aq = __builtin_fmaf(xv[q].y, xv[q].y, aq);
            aq = __builtin_fmaf(xv[q].z, xv[q].z, aq);
            aq = __builtin_fmaf(xv[q].w, xv[q].w, aq);
        }
        part[(size_t)E * G + g] = aq;
    }
    if (g == 0 && tid == 0) {
        uint32_t v = __hip_atomic_load(ctl + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int i = 0; i < n_layers; i++) v = next_gen(v);
        __hip_atomic_store(ctl + 1, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ================================================================ grouped
// Batched decode / prefill: the (token, slot) pairs of a layer are grouped
// by expert, so each selected expert's weights stream once for all of its
// tokens.  Per layer:
//
//   k_route          raw router dots (as above)
//   k_route_q8       grid (T): routing of token t (route_token), its top-k
//                    ids and weights, and Q8_0((x_t * s_t) * g) to global
//   k_group          one block: per-expert counts, offsets, and the entry
//                    list (entry i = t * k + j) of every expert
//   k_gateup_grouped grid (I/32, E): rows [32m, 32m+32) of gate and up of
//                    expert e for every entry of its group, SwiGLU, Q8_0
//                    block m of h for that entry
//   k_down_grouped   grid (H/32, E): rows [32g, 32g+32) of down of expert e
//                    for every entry of its group -> D[entry][row]
//   k_combine        grid (H/1024, T): out = resid + sum_j w_j D[t*k+j] in
//                    ascending logit order
//
// The position of an entry inside its group comes from LDS atomics and is
// not deterministic, but every (token, expert) product is computed by the
// same steps wherever it sits, and the combine visits the experts of a
// token in its own slot order, so every output is deterministic and equal
// to the per-token path bit for bit.

template <int N>
TG_DEV void scan_256_n(int (&v)[N], int n, int *tmp);

// The work items of the placed lists (k_group<false, true>'s, built by the
// last k_route_q8 block): thread e < E takes expert e's count (from the
// device-scope counts every block added to), clears it, and lists its items
// of at most G.ch entries from e * T in both lists.  Every thread calls it.
TG_DEV void route_group_items(const RouteGroup &G, int E, int T, int32_t *ecnt, int *tmp) {
    const int tid = threadIdx.x, ch = G.ch;
    if (G.rdy)
        for (int i = tid; i < G.wmax; i += RO_THREADS) G.rdy[i] = 0;
    int c = 0;
    if (tid < E) {
        const int v = __hip_atomic_load(ecnt + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        c = v < T ? v : T;  // never past the list
        __hip_atomic_store(ecnt + tid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    int sv[2] = {c, (c + ch - 1) / ch};
    scan_256_n<2>(sv, E, tmp);
    if (tid < E) {
        const int o = sv[0], bg = sv[1], ng = (c + ch - 1) / ch, ob = tid * T;
        G.offsets[tid] = o;
        G.counts[tid] = c;
        for (int i = 0; i < ng && bg + i < G.wmax; i++) {
            const int it3[3] = {tid, ob + i * ch, c - i * ch < ch ? c - i * ch : ch};
#pragma unroll
            for (int q = 0; q < 3; q++) {
                G.work[3 * (size_t)(bg + i) + q] = it3[q];
                G.work[3 * ((size_t)G.wmax + bg + i) + q] = it3[q];
            }
        }
        if (tid == E - 1) {
            G.offsets[E] = o + c;
            const int nw = bg + ng < G.wmax ? bg + ng : G.wmax;
            G.work_n[0] = nw;
            G.work_n[1] = nw;
        }
    }
}

// raw: the router dots [T][E], or (chains != null) the group chains of
// k_route_chains [G][T][E], which thread e adds in ascending group order
// first (the same sums as k_route's).
template <bool CHAINS, int NP>
__global__ __launch_bounds__(RO_THREADS) void k_route_q8(const float *__restrict__ raw, const float *__restrict__ chains,
                                                         int T, const float *__restrict__ x,
                                                         const float *__restrict__ gn, int E, int H, int k, float eps,
                                                         int32_t *__restrict__ idx,
                                                         float *__restrict__ w, int8_t *__restrict__ xq,
                                                         float *__restrict__ xd, int *__restrict__ xs,
                                                         int32_t *__restrict__ ecnt, int32_t *__restrict__ ent_cap,
                                                         RouteGroup G) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float rsum[RO_THREADS];
    RouteLds L = route_lds(smem, H);
    const int t = blockIdx.x, tid = threadIdx.x, nbH = H / QK;
    const float *rawt = raw + (size_t)t * E;
    float r0 = 0.0f;
    if (!CHAINS && tid < E) r0 = rawt[tid];  // in flight with x
    float xv[NP][8];
    route_x_load<NP>(x + (size_t)t * H, H, xv);  // in flight with the chain loads
    if constexpr (CHAINS) {
        if (tid < E) {
            const int G = H / RG;
            const float *cp = chains + (size_t)t * E + tid;
            const size_t gs = (size_t)T * E;
            float tot = 0.0f;
            for (int g0 = 0; g0 < G; g0 += 64) {  // 64 loads in flight, then the adds in order
                float cv[64];
#pragma unroll
                for (int u = 0; u < 64; u++) cv[u] = cp[(size_t)min(g0 + u, G - 1) * gs];
#pragma unroll
                for (int u = 0; u < 64; u++)
                    if (g0 + u < G) tot = tot + cv[u];
            }
            rsum[tid] = tot;
        }
        __syncthreads();
        rawt = rsum;
    }
    route_token<NP>(nullptr, CHAINS ? rawt : nullptr, E, H, k, eps, xv, L.xf, L.gss, L.slog, L.keys, L.sidx, L.sred, r0);
    if (tid < WAVE) {  // wave 0: lane i the weight of slot k - 1 - i (one exp and one division per lane)
        const float wj = topk_softmax_lane(L.slog, L.sidx, k);
        if (tid < k) {
            const int j = k - 1 - tid;
            idx[(size_t)t * k + j] = L.sidx[j];
            w[(size_t)t * k + j] = wj;
            if (ent_cap) {  // entry t k + j into its expert's list of capacity T, in arrival order
                const int e = L.sidx[j];
                const int pos = atomicAdd(ecnt + e, 1);
                // at most T tokens pick an expert, so pos < T when the count
                // started at zero (a call cut short could leave it nonzero:
                // never write past the list)
                if (pos < T) ent_cap[(size_t)e * T + pos] = t * k + j;
            }
        }
    }
    const float sc = L.sred[0];
#pragma unroll
    for (int ps = 0; ps < NP; ps++) {
        const int i0 = ps * RO_THREADS * 8 + tid * 8;
        if (ps * RO_THREADS * 8 < H) {
            float v[8];
            float4 ga = make_float4(0.f, 0.f, 0.f, 0.f), gb = ga;
            if (i0 < H) {
                ga = *reinterpret_cast<const float4 *>(gn + i0);
                gb = *reinterpret_cast<const float4 *>(gn + i0 + 4);
            }
            const float g8[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
            for (int c = 0; c < 8; c++) v[c] = (xv[ps][c] * sc) * g8[c];
            q8_group8(v, i0 < H, i0, xq + (size_t)t * H, xd + (size_t)t * nbH, xs + (size_t)t * nbH);
        }
    }
    if (G.arrive) {  // uniform: the last block to finish builds the work items
        __shared__ int last;
        __shared__ int tmp[4 * 2];
        __syncthreads();  // this block's placements are done (their atomics returned)
        if (tid == 0)
            last = __hip_atomic_fetch_add(G.arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                   (uint32_t)(T - 1);
        __syncthreads();
        if (last) {
            if (tid == 0) __hip_atomic_store(G.arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            route_group_items(G, E, T, ecnt, tmp);
        }
    }
}

constexpr int GR_THREADS = 1024;
constexpr int GR_PER = 16;  // entries per thread per pass of k_group
constexpr int GR_LDS_ENTRIES = 16384;  // entry lists staged in LDS up to this many entries

// Exclusive prefix sums of N ints per thread over threads 0..255 (threads
// >= n count as 0) with one pair of barriers: a shuffle scan per wave and
// the wave totals in LDS (tmp[4 * N]).  Every thread of the block calls it.
template <int N>
TG_DEV void scan_256_n(int (&v)[N], int n, int *tmp) {
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), wv = tid / WAVE;
    int x[N];
#pragma unroll
    for (int j = 0; j < N; j++) x[j] = tid < n ? v[j] : 0;
    for (int o = 1; o < WAVE; o <<= 1) {
#pragma unroll
        for (int j = 0; j < N; j++) {
            const int y = __shfl_up(x[j], o, WAVE);
            if (lane >= o) x[j] += y;
        }
    }
    if (tid < 4 * WAVE && lane == WAVE - 1)
#pragma unroll
        for (int j = 0; j < N; j++) tmp[wv * N + j] = x[j];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < N; j++) {
        int base = 0;
        for (int i = 0; i < wv && i < 4; i++) base += tmp[i * N + j];
        v[j] = x[j] - (tid < n ? v[j] : 0) + base;
    }
    __syncthreads();
}

// Work list: the entries of each expert cut into chunks of at most `ch`
// (gate/up) and `chd` (down) entries; item w = (expert, first entry, count)
// in work[3 * w ..], the number of items in work_n[0] (gate/up) and
// work_n[1] (down; its items start at work + 3 * wmax).  Thread e handles
// expert e: its count, offset and work items come from block scans.  SORT:
// items are listed by size class, largest first (full chunks, then
// remainders of more than half, more than a quarter, the rest), since blocks
// are dispatched in item order and the short ones then fill the tail of the
// grid; otherwise each expert's items follow one another in expert order.
// PLACED: the entries are already in per-expert lists of capacity cap
// (entries[e * cap + i], placed by k_route_q8) and ecnt[e] holds their
// counts: only the work items are built (items of expert e start at e * cap)
// and ecnt is cleared for the next layer.
// Work items of both lists (chunks of ch entries for gate/up, chd for down)
// listed by size class, largest first: full chunks, then the remainders of
// more than half, more than a quarter, the rest (blocks are dispatched in
// item order, so the short ones fill the tail of the grid).  Thread e < E
// holds expert e's count c.  Items of expert e start at its offset among all
// entries, or (cap > 0: lists of capacity cap) at e * cap.  Writes counts,
// offsets, the items and work_n; returns the thread's offset.  Every thread
// of the block calls it (threads 0..255 take part in the scans).
TG_DEV int group_items_sorted(int c, int E, int ch, int chd, int wmax, int cap, int32_t *__restrict__ counts,
                              int32_t *__restrict__ offsets, int32_t *__restrict__ work,
                              int32_t *__restrict__ work_n, int *tmp9, int *cls_tot) {
    const int tid = threadIdx.x;
    // per list (chunk size): full chunks, then the remainder in its class;
    // the counts and the class flags of both lists in one scan
    int nf[2], rr[2], cl[2];
    for (int lst = 0; lst < 2; lst++) {
        const int chk = lst ? chd : ch;
        nf[lst] = c / chk;
        rr[lst] = c - nf[lst] * chk;
        cl[lst] = rr[lst] == 0 ? -1 : (4 * rr[lst] > 2 * chk ? 0 : (4 * rr[lst] > chk ? 1 : 2));
    }
    int sv[9] = {c, nf[0], cl[0] == 0, cl[0] == 1, cl[0] == 2, nf[1], cl[1] == 0, cl[1] == 1, cl[1] == 2};
    int sc[9];
#pragma unroll
    for (int j = 0; j < 9; j++) sc[j] = sv[j];
    scan_256_n<9>(sc, E, tmp9);
    const int o = sc[0], ob = cap > 0 ? tid * cap : o;  // ob: the expert's first entry
    if (tid < E) {
        offsets[tid] = o;
        counts[tid] = c;
        if (tid == E - 1) {
            offsets[E] = o + c;
            // class totals (exclusive scan + own value)
            for (int j = 0; j < 8; j++) cls_tot[j] = sc[1 + j] + sv[1 + j];
        }
    }
    __syncthreads();
    for (int lst = 0; lst < 2; lst++) {
        const int chk = lst ? chd : ch, nfull = nf[lst], r = rr[lst], cls = cl[lst];
        const int *tot4 = cls_tot + 4 * lst;
        const int bf = sc[1 + 4 * lst], b0 = sc[2 + 4 * lst], b1 = sc[3 + 4 * lst], b2 = sc[4 + 4 * lst];
        const int base_r = cls == 0 ? tot4[0] + b0 : cls == 1 ? tot4[0] + tot4[1] + b1 : tot4[0] + tot4[1] + tot4[2] + b2;
        int32_t *wl = work + 3 * (size_t)(lst ? wmax : 0);
        if (tid < E) {
            for (int i = 0; i < nfull && bf + i < wmax; i++) {
                int32_t *it = wl + 3 * (size_t)(bf + i);
                it[0] = tid;
                it[1] = ob + i * chk;
                it[2] = chk;
            }
            if (cls >= 0 && base_r < wmax) {
                int32_t *it = wl + 3 * (size_t)base_r;
                it[0] = tid;
                it[1] = ob + nfull * chk;
                it[2] = r;
            }
        }
        if (tid == 0) {
            const int tot = tot4[0] + tot4[1] + tot4[2] + tot4[3];
            work_n[lst] = tot < wmax ? tot : wmax;
        }
    }
    __syncthreads();
    return o;
}

template <bool SORT, bool PLACED = false>
__global__ __launch_bounds__(GR_THREADS) void k_group(const int32_t *__restrict__ idx, int n, int E, int ch, int chd,
                                                      int wmax, int32_t *__restrict__ counts,
                                                      int32_t *__restrict__ offsets, int32_t *__restrict__ entries,
                                                      int32_t *__restrict__ work, int32_t *__restrict__ work_n,
                                                      int32_t *__restrict__ ecnt, int cap,
                                                      int32_t *__restrict__ rdy) {
    __shared__ int cnt[MAX_E], off[MAX_E + 1], fill[MAX_E], tmp9[4 * 9], cls_tot[8];
    const int tid = threadIdx.x;
    if (rdy)  // the fused gate/up + down launch's per-item counts
        for (int i = tid; i < wmax; i += GR_THREADS) rdy[i] = 0;
    for (int e = tid; e < E; e += GR_THREADS) {
        cnt[e] = 0;
        fill[e] = 0;
    }
    if constexpr (PLACED) {
        if (tid < E) {
            const int v = ecnt[tid];
            cnt[tid] = v < cap ? v : cap;  // never past the list
            ecnt[tid] = 0;
        }
        n = 0;  // no entry to count or list
    }
    __syncthreads();
    // GR_PER entries per thread per pass, loaded together before the atomics
    // (one load latency per pass rather than one per entry); the first
    // pass's ids stay in registers for the entry lists below
    int ev0[GR_PER];
    for (int base = 0; base < n; base += GR_THREADS * GR_PER) {
        int ev[GR_PER];
#pragma unroll
        for (int u = 0; u < GR_PER; u++) {
            const int i = base + u * GR_THREADS + tid;
            ev[u] = i < n ? idx[i] : -1;
            if (base == 0) ev0[u] = ev[u];
        }
#pragma unroll
        for (int u = 0; u < GR_PER; u++) {
            if (base + u * GR_THREADS + tid < n) {
                const int e = ev[u] < 0 ? 0 : (ev[u] >= E ? E - 1 : ev[u]);  // never index outside the table
                atomicAdd(&cnt[e], 1);
            }
        }
    }
    __syncthreads();
    const int c = tid < E ? cnt[tid] : 0;
    if constexpr (!SORT) {
        int sv[3] = {c, (c + ch - 1) / ch, (c + chd - 1) / chd};
        scan_256_n<3>(sv, E, tmp9);
        const int o = sv[0], bg = sv[1], bd = sv[2], ng = (c + ch - 1) / ch, nd = (c + chd - 1) / chd;
        const int ob = PLACED ? tid * cap : o;  // the expert's first entry
        if (tid < E) {
            off[tid] = o;
            offsets[tid] = o;
            counts[tid] = c;
            for (int i = 0; i < ng && bg + i < wmax; i++) {
                int32_t *it = work + 3 * (size_t)(bg + i);
                it[0] = tid;
                it[1] = ob + i * ch;
                it[2] = c - i * ch < ch ? c - i * ch : ch;
            }
            for (int i = 0; i < nd && bd + i < wmax; i++) {
                int32_t *it = work + 3 * ((size_t)wmax + bd + i);
                it[0] = tid;
                it[1] = ob + i * chd;
                it[2] = c - i * chd < chd ? c - i * chd : chd;
            }
            if (tid == E - 1) {
                offsets[E] = o + c;
                work_n[0] = bg + ng < wmax ? bg + ng : wmax;
                work_n[1] = bd + nd < wmax ? bd + nd : wmax;
            }
        }
        __syncthreads();
    } else {
        const int o = group_items_sorted(c, E, ch, chd, wmax, PLACED ? cap : 0, counts, offsets, work, work_n, tmp9,
                                         cls_tot);
        if (tid < E) off[tid] = o;
        __syncthreads();
    }
    // entry lists: built in LDS when they fit (the dynamic buffer holds n
    // ints), then written out in order, coalesced; scattered 4-byte stores
    // to global memory cost one cache line each
    extern __shared__ int ent_l[];
    const bool in_lds = n <= GR_LDS_ENTRIES;
    for (int base = 0; base < n; base += GR_THREADS * GR_PER) {
        int ev[GR_PER];
#pragma unroll
        for (int u = 0; u < GR_PER; u++) {
            const int i = base + u * GR_THREADS + tid;
            ev[u] = base == 0 ? ev0[u] : (i < n ? idx[i] : -1);
        }
#pragma unroll
        for (int u = 0; u < GR_PER; u++) {
            const int i = base + u * GR_THREADS + tid;
            if (i < n) {
                const int e = ev[u] < 0 ? 0 : (ev[u] >= E ? E - 1 : ev[u]);
                const int pos = atomicAdd(&fill[e], 1);
                if (in_lds)
                    ent_l[off[e] + pos] = i;
                else
                    entries[off[e] + pos] = i;
            }
        }
    }
    if (in_lds) {
        __syncthreads();
        for (int i = tid; i < n; i += GR_THREADS) entries[i] = ent_l[i];
    }
}

// Many entries (prefill): the entries are placed in per-expert lists of
// capacity cap by many blocks (the role of k_route_q8's placement below 128
// tokens, without its contention): each block counts its PL_THREADS * PL_PER
// entries per expert in LDS, reserves each expert's range with one
// device-scope atomic on ecnt[e] and writes its entries there; the last
// block to finish (one arrival count, G.arrive) builds the work items of
// both lists in k_group's size order from the counts and clears them.
// Positions inside a list depend on the order of the atomics, as in k_group.
constexpr int PL_THREADS = 256, PL_PER = 4;

__global__ __launch_bounds__(PL_THREADS) void k_place(const int32_t *__restrict__ idx, int n, int E, int cap,
                                                      int32_t *__restrict__ ecnt, int32_t *__restrict__ ent_cap,
                                                      RouteGroup G) {
    __shared__ int lcnt[MAX_E], lbase[MAX_E];
    const int tid = threadIdx.x, b0 = (int)blockIdx.x * PL_THREADS * PL_PER;
    for (int e = tid; e < E; e += PL_THREADS) lcnt[e] = 0;
    int ev[PL_PER], lp[PL_PER];
#pragma unroll
    for (int u = 0; u < PL_PER; u++) {
        const int i = b0 + u * PL_THREADS + tid;
        const int v = i < n ? idx[i] : -1;
        ev[u] = i < n ? (v < 0 ? 0 : (v >= E ? E - 1 : v)) : -1;  // never index outside the table
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < PL_PER; u++)
        if (ev[u] >= 0) lp[u] = atomicAdd(&lcnt[ev[u]], 1);
    __syncthreads();
    for (int e = tid; e < E; e += PL_THREADS)
        if (lcnt[e]) lbase[e] = atomicAdd(ecnt + e, lcnt[e]);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < PL_PER; u++) {
        if (ev[u] >= 0) {
            const int pos = lbase[ev[u]] + lp[u];
            // at most cap entries per expert when the counts started at zero
            // (a call cut short could leave them nonzero: never write past the list)
            if (pos < cap) ent_cap[(size_t)ev[u] * cap + pos] = b0 + u * PL_THREADS + tid;
        }
    }
    __shared__ int last, tmp9[4 * 9], cls_tot[8];
    __syncthreads();  // this block's reservations are done (their atomics returned)
    if (tid == 0)
        last = __hip_atomic_fetch_add(G.arrive, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
    __syncthreads();
    if (!last) return;  // uniform over the block
    if (tid == 0) __hip_atomic_store(G.arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (G.rdy)
        for (int i = tid; i < G.wmax; i += PL_THREADS) G.rdy[i] = 0;
    int c = 0;
    if (tid < E) {
        const int v = __hip_atomic_load(ecnt + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        c = v < cap ? v : cap;  // never past the list
        __hip_atomic_store(ecnt + tid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    group_items_sorted(c, E, G.ch, G.ch, G.wmax, cap, G.counts, G.offsets, G.work, G.work_n, tmp9, cls_tot);
}

// Tokens (entries) per chunk of the grouped kernels, from an LDS budget.
constexpr size_t GRP_LDS_BUDGET = 72 * 1024;

__host__ __device__ inline int gu_chunk(int nbH) {
    size_t per = (size_t)64 * (round4(nbH) + 4) * 4 + (size_t)nbH * QK + 8 * (size_t)round4(nbH);
    int tc = (int)(GRP_LDS_BUDGET / per);
    return tc < 1 ? 1 : (tc > 8 ? 8 : tc);
}

__host__ __device__ inline size_t gu_grouped_lds(int nbH) {
    const int tc = gu_chunk(nbH);
    return (size_t)tc * ((size_t)64 * (round4(nbH) + 4) * 4 + (size_t)nbH * QK + 8 * (size_t)round4(nbH)) +
           4 * (size_t)tc * 64 + 4 * 8;
}

template <int NT, int UNR>
__global__ __launch_bounds__(NT) void k_gateup_grouped(const uint8_t *__restrict__ layer_pl, Shape s,
                                                               const int32_t *__restrict__ work,
                                                               const int32_t *__restrict__ work_n,
                                                               const int32_t *__restrict__ entries,
                                                               const int8_t *__restrict__ xq,
                                                               const float *__restrict__ xd,
                                                               const int *__restrict__ xs, int8_t *__restrict__ hq,
                                                               float *__restrict__ hd, int *__restrict__ hs) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int wi = blockIdx.y, m = blockIdx.x, tid = threadIdx.x;
    if (wi >= work_n[0]) return;
    const int e = work[3 * wi], o = work[3 * wi + 1], c = work[3 * wi + 2];
    const int nb = s.nbH, nbp = round4(nb), ust = nbp + 4, H = s.H, k = s.k, tc = gu_chunk(nb);
    float *U = reinterpret_cast<float *>(smem);                         // [tc][64][ust]
    int8_t *lq = reinterpret_cast<int8_t *>(U + (size_t)tc * 64 * ust); // [tc][H]
    float *ld = reinterpret_cast<float *>(lq + (size_t)tc * H);         // [tc][nbp]
    int *ls = reinterpret_cast<int *>(ld + (size_t)tc * nbp);           // [tc][nbp]
    float *D = reinterpret_cast<float *>(ls + (size_t)tc * nbp);        // [tc][64]
    int *ent = reinterpret_cast<int *>(D + (size_t)tc * 64);            // [8]

    // gate and up rows [32m, 32m+32) of expert e, all issued first
    const uint8_t *ex = layer_pl + (size_t)e * s.EB;
    const size_t ntb = (size_t)s.I * nb;
    const int items = 64 * nb;
    uint4 wv[UNR];
    uint32_t dv[UNR];
#pragma unroll
    for (int u = 0; u < UNR; u++) {  // clamped, unbranched loads (as k_gateup)
        const int p = min(u * NT + tid, items - 1);
        const int rd = (int)fdiv((uint32_t)p, s.divH), b = p - rd * nb;
        const uint8_t *tb = ex + (size_t)(rd >> 5) * s.GB;
        const size_t ob = (size_t)(m * 32 + (rd & 31)) * nb + b;
        wv[u] = reinterpret_cast<const uint4 *>(tb)[ob];
        dv[u] = reinterpret_cast<const uint16_t *>(tb + ntb * 16)[ob];
    }
    for (int c0 = 0; c0 < c; c0 += tc) {
        const int nt = c - c0 < tc ? c - c0 : tc;
        if (tid < nt) ent[tid] = entries[o + c0 + tid];
        __syncthreads();
        // Q8_0 x of the chunk's tokens -> LDS
        for (int q = 0; q < nt; q++) {
            const int t = ent[q] / k;
            const int *src = reinterpret_cast<const int *>(xq + (size_t)t * H);
            int *dst = reinterpret_cast<int *>(lq + (size_t)q * H);
            for (int i = tid; i < H / 4; i += NT) dst[i] = src[i];
            for (int b = tid; b < nb; b += NT) {
                ld[q * nbp + b] = xd[(size_t)t * nb + b];
                ls[q * nbp + b] = xs[(size_t)t * nb + b];
            }
        }
        __syncthreads();
        for (int q = 0; q < nt; q++) {
            const int8_t *xqq = lq + (size_t)q * H;
            const int *lsq = ls + q * nbp;
            float *Uq = U + (size_t)q * 64 * ust;
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                const int p = u * NT + tid;
                if (p < items) {
                    const int rd = (int)fdiv((uint32_t)p, s.divH), b = p - rd * nb;
                    const int S = dot_q4_q8(wv[u], reinterpret_cast<const int *>(xqq + b * QK)) - 8 * lsq[b];
                    Uq[rd * ust + b] = (float)S * h2f(dv[u]);
                }
            }
        }
        __syncthreads();
        for (int r = tid; r < nt * 64; r += NT) {
            const int q = r >> 6;
            D[r] = chain4(U + (size_t)r * ust, ld + q * nbp, nb);
        }
        __syncthreads();
        // h rows -> Q8_0 block m of each entry (32 lanes per entry)
        {
            const int q = tid >> 5, rr = tid & 31;
            const bool on = q < nt;
            const float hv = on ? silu_mul(D[q * 64 + rr], D[q * 64 + 32 + rr]) : 0.0f;
            float dq; int qsum; uint16_t dh;
            const int qv = q8_lane(hv, dq, qsum, dh);
            if (on) {
                const int i = ent[q];
                hq[(size_t)i * s.I + m * 32 + rr] = (int8_t)qv;
                if (rr == 0) {
                    hd[(size_t)i * s.nbI + m] = dq;
                    hs[(size_t)i * s.nbI + m] = qsum;
                }
            }
        }
        __syncthreads();
    }
}

__host__ __device__ inline int dn_chunk(int nbI, int I) {
    size_t per = (size_t)32 * (round4(nbI) + 4) * 4 + (size_t)I + 8 * (size_t)round4(nbI);
    int tc = (int)(GRP_LDS_BUDGET / per);
    return tc < 1 ? 1 : (tc > 16 ? 16 : tc);
}

__host__ __device__ inline size_t dn_grouped_lds(int nbI, int I) {
    const int tc = dn_chunk(nbI, I);
    return (size_t)tc * ((size_t)32 * (round4(nbI) + 4) * 4 + (size_t)I + 8 * (size_t)round4(nbI)) + 4 * 16;
}

template <int UNR>
__global__ __launch_bounds__(RO_THREADS) void k_down_grouped(const uint8_t *__restrict__ layer_pl, Shape s,
                                                             const int32_t *__restrict__ work,
                                                             const int32_t *__restrict__ work_n,
                                                             const int32_t *__restrict__ entries,
                                                             const int8_t *__restrict__ hq,
                                                             const float *__restrict__ hd,
                                                             const int *__restrict__ hs, float *__restrict__ D) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int wi = blockIdx.y, g = blockIdx.x, tid = threadIdx.x;
    if (wi >= work_n[1]) return;
    const int e = work[3 * wi], o = work[3 * wi + 1], c = work[3 * wi + 2];
    const int nb = s.nbI, nbp = round4(nb), ust = nbp + 4, I = s.I, tc = dn_chunk(nb, I);
    float *U = reinterpret_cast<float *>(smem);                          // [tc][32][ust]
    int8_t *lq = reinterpret_cast<int8_t *>(U + (size_t)tc * 32 * ust);  // [tc][I]
    float *ld = reinterpret_cast<float *>(lq + (size_t)tc * I);          // [tc][nbp]
    int *ls = reinterpret_cast<int *>(ld + (size_t)tc * nbp);            // [tc][nbp]
    int *ent = reinterpret_cast<int *>(ls + (size_t)tc * nbp);           // [16]

    const uint8_t *tb = layer_pl + (size_t)e * s.EB + 2 * s.GB;
    const size_t ntb = (size_t)s.H * nb;
    const int items = 32 * nb;
    uint4 wv[UNR];
    uint32_t dv[UNR];
#pragma unroll
    for (int u = 0; u < UNR; u++) {  // clamped, unbranched loads (as k_gateup)
        const size_t ob = (size_t)g * 32 * nb + min(u * RO_THREADS + tid, items - 1);
        wv[u] = reinterpret_cast<const uint4 *>(tb)[ob];
        dv[u] = reinterpret_cast<const uint16_t *>(tb + ntb * 16)[ob];
    }
    for (int c0 = 0; c0 < c; c0 += tc) {
        const int nt = c - c0 < tc ? c - c0 : tc;
        if (tid < nt) ent[tid] = entries[o + c0 + tid];
        __syncthreads();
        for (int q = 0; q < nt; q++) {
            const int i = ent[q];
            const int *src = reinterpret_cast<const int *>(hq + (size_t)i * I);
            int *dst = reinterpret_cast<int *>(lq + (size_t)q * I);
            for (int a = tid; a < I / 4; a += RO_THREADS) dst[a] = src[a];
            for (int b = tid; b < nb; b += RO_THREADS) {
                ld[q * nbp + b] = hd[(size_t)i * nb + b];
                ls[q * nbp + b] = hs[(size_t)i * nb + b];
            }
        }
        __syncthreads();
        for (int q = 0; q < nt; q++) {
            const int8_t *hqq = lq + (size_t)q * I;
            const int *lsq = ls + q * nbp;
            float *Uq = U + (size_t)q * 32 * ust;
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                const int p = u * RO_THREADS + tid;
                if (p < items) {
                    const int row = (int)fdiv((uint32_t)p, s.divI), b = p - row * nb;
                    const int S = dot_q4_q8(wv[u], reinterpret_cast<const int *>(hqq + b * QK)) - 8 * lsq[b];
                    Uq[row * ust + b] = (float)S * h2f(dv[u]);
                }
            }
        }
        __syncthreads();
        for (int r = tid; r < nt * 32; r += RO_THREADS) {
            const int q = r >> 5;
            D[(size_t)ent[q] * s.H + g * 32 + (r & 31)] = chain4(U + (size_t)r * ust, ld + q * nbp, nb);
        }
        __syncthreads();
    }
}

// One column per thread: for out / resid pointers that are not 16-byte
// aligned.
__global__ __launch_bounds__(256) void k_combine1(const float *__restrict__ D, const float *__restrict__ w, int H,
                                                  int k, const float *resid, float *out) {
    const int t = blockIdx.y, r = blockIdx.x * 256 + threadIdx.x;
    if (r >= H) return;
    float acc = 0.0f;
    for (int jj = k - 1; jj >= 0; jj--)
        acc = __builtin_fmaf(w[(size_t)t * k + jj], D[((size_t)t * k + jj) * H + r], acc);
    out[(size_t)t * H + r] = resid ? resid[(size_t)t * H + r] + acc : acc;
}

// Four columns per thread (H % 4 == 0): the k rows' float4 loads are issued
// together, then folded in slot order k-1 .. 0 per column, as k_combine1.
__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ D, const float *__restrict__ w, int H,
                                                 int k, const float *resid, float *out) {
    const int t = blockIdx.y, c4 = blockIdx.x * 256 + threadIdx.x, H4 = H >> 2;
    if (c4 >= H4) return;
    const float4 *D4 = reinterpret_cast<const float4 *>(D + (size_t)t * k * H) + c4;
    float4 v[MAX_K];
#pragma unroll
    for (int jj = 0; jj < MAX_K; jj++)
        if (jj < k) v[jj] = D4[(size_t)jj * H4];
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int jj = MAX_K - 1; jj >= 0; jj--) {
        if (jj < k) {
            const float wj = w[(size_t)t * k + jj];
            acc.x = __builtin_fmaf(wj, v[jj].x, acc.x);
            acc.y = __builtin_fmaf(wj, v[jj].y, acc.y);
            acc.z = __builtin_fmaf(wj, v[jj].z, acc.z);
            acc.w = __builtin_fmaf(wj, v[jj].w, acc.w);
        }
    }
    if (resid) {
        const float4 r = reinterpret_cast<const float4 *>(resid + (size_t)t * H)[c4];
        acc = make_float4(r.x + acc.x, r.y + acc.y, r.z + acc.z, r.w + acc.w);
    }
    reinterpret_cast<float4 *>(out + (size_t)t * H)[c4] = acc;
}

// ================================================================ launchers
static inline unsigned cdiv(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }

// Kernels whose LDS exceeds the 64 KiB default opt in to more (gfx950 has
// 160 KiB per CU).
static hipError_t allow_lds(const void *fn, size_t bytes) {
    if (bytes <= 65536) return hipSuccess;
    return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

bool decode_shape_ok(const Shape &s) {
    return s.H <= RO_MAXPASS * RO_THREADS * 8 && s.H / RG <= RT_THREADS && s.H / 8 <= GU_THREADS &&
           s.nbH <= GU_THREADS && 2 * GU_ROWS * s.nbH <= 16 * GU_THREADS && gateup_lds_bytes(s.H, s.nbH) <= 160 * 1024 &&
           s.k * DN_RD * s.nbI <= 16 * DN_THREADS && down_lds_bytes(s.k, s.I, s.nbI) <= 160 * 1024 &&
           s.E < RO_THREADS && s.E <= MAX_E && s.E % 4 == 0 && s.k <= MAX_K;
}

hipError_t launch_route(const float *Wr, const float *x, int T, int E, int H, float *raw, hipStream_t st) {
    if (T >= 128 && (H / RG) % 8 == 0) {
        TG_LAUNCH(k_route_tiled<8>, dim3(cdiv((size_t)T, RTT_T), cdiv((size_t)E, RTT_E)), dim3(512), 0, st, Wr, x, T,
                  E, H, raw);
    } else if (T >= 128 && (H / RG) % RT_CH == 0) {
        TG_LAUNCH(k_route_tiled<4>, dim3(cdiv((size_t)T, RTT_T), cdiv((size_t)E, RTT_E)), dim3(256), 0, st, Wr, x, T,
                  E, H, raw);
    } else if (T >= RS_T && (H / RG) % (2 * RS_PARTS) == 0 && route_small_lds(H) <= 64 * 1024) {
        const size_t lds = route_small_lds(H);
        hipError_t e = allow_lds((const void *)k_route_small, lds);
        if (e != hipSuccess) return e;
        TG_LAUNCH(k_route_small, dim3(cdiv((size_t)T, RS_T), cdiv((size_t)E, RS_E)), dim3(1024), lds, st,
                           Wr, x, T, E, H, raw);
    } else {
        TG_LAUNCH(k_route, dim3(E, cdiv((size_t)T, RT_TOK)), dim3(RT_THREADS), 0, st, Wr, x, T, E, H, raw);
    }
    return hipGetLastError();
}

hipError_t launch_topk(const float *raw, const float *x, int T, int E, int H, int k, float eps, float *logits,
                       int32_t *idx, float *w, hipStream_t st) {
    size_t lds = route_lds_bytes(H);
    hipError_t e = allow_lds((const void *)k_topk, lds);
    if (e != hipSuccess) return e;
    TG_LAUNCH(k_topk, dim3(T), dim3(RO_THREADS), lds, st, raw, x, E, H, k, eps, logits, idx, w);
    return hipGetLastError();
}

hipError_t launch_route_dec(const float *Wr, const float *x, const float *gn, int T, const Shape &s, float eps,
                            uint64_t *lw, uint32_t *ctl, uint32_t *err, int32_t *idx, float *w, int8_t *xq, float *xd,
                            int *xs, hipStream_t st) {
    if (!decode_shape_ok(s)) return hipErrorInvalidValue;
    TG_LAUNCH(k_route_dec, dim3(s.E, T), dim3(RD_THREADS), 0, st, Wr, x, gn, s.E, s.H, s.k, eps, lw, ctl, err, idx,
                       w, xq, xd, xs);
    return hipGetLastError();
}

template <int UNR>
static hipError_t gateup_go(const uint8_t *layer_pl, const Shape &s, int T, const int32_t *idx, const int8_t *xq,
                            const float *xd, const int *xs, int8_t *hq, float *hd, int *hs, hipStream_t st) {
    const size_t lds = gateup_lds_bytes(s.H, s.nbH);
    hipError_t e = allow_lds((const void *)k_gateup<UNR>, lds);
    if (e != hipSuccess) return e;
    TG_LAUNCH(k_gateup<UNR>, dim3(s.I / GU_ROWS, s.k, T), dim3(GU_THREADS), lds, st, layer_pl, s, idx, xq,
                       xd, xs, hq, hd, hs);
    return hipGetLastError();
}

hipError_t launch_gateup(const uint8_t *layer_pl, const Shape &s, int T, const int32_t *idx, const int8_t *xq,
                         const float *xd, const int *xs, int8_t *hq, float *hd, int *hs, hipStream_t st) {
    if (!decode_shape_ok(s)) return hipErrorInvalidValue;
    const int per = (int)cdiv((size_t)2 * GU_ROWS * s.nbH, GU_THREADS);
    if (per <= 1) return gateup_go<1>(layer_pl, s, T, idx, xq, xd, xs, hq, hd, hs, st);
    if (per <= 2) return gateup_go<2>(layer_pl, s, T, idx, xq, xd, xs, hq, hd, hs, st);
    if (per <= 4) return gateup_go<4>(layer_pl, s, T, idx, xq, xd, xs, hq, hd, hs, st);
    if (per <= 8) return gateup_go<8>(layer_pl, s, T, idx, xq, xd, xs, hq, hd, hs, st);
    return gateup_go<16>(layer_pl, s, T, idx, xq, xd, xs, hq, hd, hs, st);
}

template <int UNR>
static hipError_t down_go(const uint8_t *layer_pl, const Shape &s, int T, const int32_t *idx, const float *w,
                          const int8_t *hq, const float *hd, const int *hs, const float *resid, float *out,
                          hipStream_t st) {
    const size_t lds = down_lds_bytes(s.k, s.I, s.nbI);
    hipError_t e = allow_lds((const void *)k_down<UNR>, lds);
    if (e != hipSuccess) return e;
    TG_LAUNCH(k_down<UNR>, dim3(s.H / DN_RD, T), dim3(DN_THREADS), lds, st, layer_pl, s, idx, w, hq, hd, hs,
                       resid, out);
    return hipGetLastError();
}

hipError_t launch_down(const uint8_t *layer_pl, const Shape &s, int T, const int32_t *idx, const float *w,
                       const int8_t *hq, const float *hd, const int *hs, const float *resid, float *out,
                       hipStream_t st) {
    if (!decode_shape_ok(s)) return hipErrorInvalidValue;
    const int per = (int)cdiv((size_t)s.k * DN_RD * s.nbI, DN_THREADS);
    if (per <= 2) return down_go<2>(layer_pl, s, T, idx, w, hq, hd, hs, resid, out, st);
    if (per <= 6) return down_go<6>(layer_pl, s, T, idx, w, hq, hd, hs, resid, out, st);
    if (per <= 12) return down_go<12>(layer_pl, s, T, idx, w, hq, hd, hs, resid, out, st);
    return down_go<16>(layer_pl, s, T, idx, w, hq, hd, hs, resid, out, st);
}

// Down rows per block: the smallest power of two that keeps the grid within
// the CU count (one resident block per CU).
static int fx_rows(const Shape &s, int n_cu) {
    int rd = 1;
    while (s.H / rd > n_cu || s.H % rd) rd *= 2;
    return rd;
}

bool experts_fused_ok(const Shape &s, int n_cu) {
    if (!decode_shape_ok(s) || n_cu <= 0) return false;
    const int rd = fx_rows(s, n_cu);
    // unroll variants that stay within 128 VGPRs without spills
    const int ug = (int)cdiv((size_t)2 * GU_ROWS * s.nbH, FX_THREADS);
    const int ud = (int)cdiv((size_t)s.k * rd * s.nbI, FX_DT);
    const bool regs = ud <= 6 && ug <= 4 && !(ug > 2 && ud > 2);
    return regs && s.H % rd == 0 && s.k * rd <= FX_THREADS && fx_lds_bytes(s, rd) <= 160 * 1024 && s.k <= MAX_K;
}

// (two parities; each holds a line per unit, or per half unit for the layer
// launch's half units: 2 HU_QS words per unit = 2 FX_QS)
size_t experts_fused_words(const Shape &s) { return 2 * 2 * (size_t)s.k * s.nbI * FX_QS; }

template <int UG, int UD>
static hipError_t experts_go(const FxArgs &A, const Shape &s, hipStream_t st) {
    const size_t lds = fx_lds_bytes(s, A.rd);
    hipError_t e = allow_lds((const void *)k_experts<UG, UD>, lds);
    if (e != hipSuccess) return e;
    TG_LAUNCH((k_experts<UG, UD>), dim3(s.H / A.rd), dim3(FX_THREADS), lds, st, A, s);
    return hipGetLastError();
}

template <int UG, int UDMAX>
static hipError_t experts_ud(const FxArgs &A, const Shape &s, hipStream_t st) {
    const int ud = (int)cdiv((size_t)s.k * A.rd * s.nbI, FX_DT);
    if (ud <= 1) return experts_go<UG, 1>(A, s, st);
    if (ud <= 2 || UDMAX <= 2) return experts_go<UG, 2>(A, s, st);
    return experts_go<UG, UDMAX>(A, s, st);
}

hipError_t launch_experts_fused(const uint8_t *layer_pl, const Shape &s, int n_cu, const int32_t *idx, const float *w,
                                const int8_t *xq, const float *xd, const int *xs, uint64_t *hw, const uint32_t *ctl,
                                uint32_t *err, const float *resid, float *out, hipStream_t st) {
    if (!experts_fused_ok(s, n_cu)) return hipErrorInvalidValue;
    const FxArgs A{layer_pl, idx, w, xq, xd, xs, hw, ctl, err, resid, out, fx_rows(s, n_cu), fault_spin_limit(),
                   g_fault_drop};
    const int ug = (int)cdiv((size_t)2 * GU_ROWS * s.nbH, FX_THREADS);
    if (ug <= 1) return experts_ud<1, 6>(A, s, st);
    if (ug <= 2) return experts_ud<2, 6>(A, s, st);
    return experts_ud<4, 2>(A, s, st);
}

// One-token layer with routing inside: rd output rows per block, the
// smallest of 8, 16, 32 that keeps the grid (H / rd blocks, one per CU at
// most, all resident at once) within the CUs.
static int ld_rows(const Shape &s, int n_cu) {
    for (int rd = 8; rd <= RG; rd *= 2)
        if (s.H % rd == 0 && s.H / rd <= n_cu) return rd;
    return 0;
}

static int ld_ud(const Shape &s, int rd) { return (int)cdiv((size_t)s.k * rd * s.nbI, FX_THREADS); }

// TG_LD_HALF=0 keeps whole units on shapes with more units than blocks
static bool ld_half_units() {
    static const bool on = [] {
        const char *v = getenv("TG_LD_HALF");
        return !(v && v[0] == '0');
    }();
    return on;
}

// dynamic LDS of the routed launch: the deep variant (<8, 6>) adds its
// staged down scales and residual rows
template <int UG, int UD>
static size_t ld_launch_lds(const Shape &s, int rd) {
    return ld_lds_bytes(s, rd) + (UG > 4 ? 4 * ((size_t)UD * FX_THREADS + WAVE) : 0);
}

static bool ld_shallow(const Shape &s, int rd) {
    return cdiv((size_t)2 * GU_ROWS * s.nbH, FX_THREADS) <= 4 && ld_ud(s, rd) <= 2;
}

bool layer_dec_ok(const Shape &s, int n_cu) {
    const int rd = n_cu > 0 ? ld_rows(s, n_cu) : 0;
    if (!rd) return false;
    const int ug = (int)cdiv((size_t)2 * GU_ROWS * s.nbH, FX_THREADS);
    const size_t lds = ld_shallow(s, rd) ? ld_launch_lds<4, 2>(s, rd) : ld_launch_lds<8, 6>(s, rd);
    return decode_shape_ok(s) && s.H % RG == 0 && (s.H / RG) % 4 == 0 && s.E * (RG / 4) <= FX_THREADS &&
           s.E <= LD_EMAX && (s.nbH & (s.nbH - 1)) == 0 && s.nbH <= 256 && s.nbI < 65536 &&
           s.E < 256 && s.k * rd <= FX_THREADS && s.H / 8 + WAVE <= FX_THREADS && ug <= 8 && ld_ud(s, rd) <= 6 &&
           RG - rd <= FX_THREADS && lds <= 160 * 1024;
}

hipError_t launch_dec_part(const float *Wr, const float *x, const Shape &s, float *part, uint32_t *ctl, int n_layers,
                           hipStream_t st) {
    TG_LAUNCH(k_dec_part, dim3(s.H / RG), dim3(256), 0, st, Wr, x, s.E, s.H, part, ctl, n_layers);
    return hipGetLastError();
}

template <int UG, int UD, bool HU, bool XS>
static hipError_t ld_go_xs(const LdArgs &A, const Shape &s, hipStream_t st) {
    const size_t lds = ld_launch_lds<UG, UD>(s, A.rd);
    hipError_t e = allow_lds((const void *)k_layer_dec<UG, UD, HU, XS>, lds);
    if (e != hipSuccess) return e;
    TG_LAUNCH((k_layer_dec<UG, UD, HU, XS>), dim3(s.H / A.rd), dim3(FX_THREADS), lds, st, A.part_in, s.E, s.H / RG,
              A, s);
    return hipGetLastError();
}

// TG_LD_XS=0 keeps the down rows of every slot in each block (each block
// then reads the h of every expert)
static bool ld_xs_enabled() {
    static const bool on = [] {
        const char *v = getenv("TG_LD_XS");
        return !(v && v[0] == '0');
    }();
    return on;
}

// The expert-sliced down: the grid splits into k slots of whole row slices
// (k RD rows each), the slice's chains fit the block, an owner's k RG slot
// values fit behind slot 0 of hq, every slot's units are polled in one pass.
static bool ld_xs_ok(const Shape &s, int rd) {
    const int nblk = s.H / rd;
    return ld_xs_enabled() && nblk % s.k == 0 && s.k * rd <= FX_THREADS && s.k * RG <= FX_THREADS &&
           (size_t)((s.I + 15) & ~15) + 4 * (size_t)s.k * RG <= (size_t)s.k * s.I && s.nbI <= FX_PT;
}

template <int UG, int UD, bool HU>
static hipError_t ld_go(const LdArgs &A, const Shape &s, hipStream_t st) {
    if (ld_xs_ok(s, A.rd)) return ld_go_xs<UG, UD, HU, true>(A, s, st);
    return ld_go_xs<UG, UD, HU, false>(A, s, st);
}

hipError_t launch_layer_dec(const uint8_t *layer_pl, const Shape &s, int n_cu, const float *x, const float *gn,
                            const float *part_in, const float *wr_next, float *part_out, uint64_t *hw, uint64_t *ow,
                            const uint32_t *ctl, uint32_t back, uint32_t *err, const float *resid, float *out,
                            int32_t *idx, float *w, float eps, hipStream_t st) {
    if (!layer_dec_ok(s, n_cu)) return hipErrorInvalidValue;
    const int rd = ld_rows(s, n_cu);
    const LdArgs A{layer_pl, x, gn, part_in, wr_next, part_out, hw, ow, ctl, back, err, resid, out, idx, w, eps, rd,
                   fault_spin_limit(), g_fault_drop};
    if (ld_shallow(s, rd)) return ld_go<4, 2, false>(A, s, st);
    // more units than blocks: half units, so every block carries the same
    // number (each half unit's items fit four loads per thread)
    const int ng = (s.I / GU_ROWS) * s.k, nblk = s.H / rd;
    if (ld_half_units() && ng > nblk && 2 * HU_ROWS * s.nbH <= 4 * FX_THREADS) return ld_go<8, 6, true>(A, s, st);
    return ld_go<8, 6, false>(A, s, st);
}

size_t dec_part_floats(const Shape &s) { return 2 * (size_t)(s.H / RG) * (s.E + 1); }
size_t dec_ow_words(const Shape &s) { return 2 * (size_t)s.k * s.H; }  // [2][k][H] (expert-sliced down)

bool grouped_shape_ok(const Shape &s) {
    return decode_shape_ok(s) && 64 * s.nbH <= 16 * 512 && 32 * s.nbI <= 16 * RO_THREADS &&
           gu_grouped_lds(s.nbH) <= 160 * 1024 && dn_grouped_lds(s.nbI, s.I) <= 160 * 1024;
}

hipError_t launch_route_q8(const float *raw, const float *chains, const float *x, const float *gn, int T, int E,
                           int H, int k, float eps, int32_t *idx, float *w, int8_t *xq, float *xd, int *xs,
                           int32_t *ecnt, int32_t *ent_cap, const RouteGroup &G, hipStream_t st) {
    if (G.arrive && (!ent_cap || !ecnt || G.ch <= 0 || G.wmax <= 0 || E > RO_THREADS || !G.counts || !G.offsets ||
                     !G.work || !G.work_n))
        return hipErrorInvalidValue;
    // x in registers: NP passes of 8 x 256 elements.  The raw-dot form (many
    // tokens, one block each) takes as few passes as H needs, so its blocks
    // need fewer registers and more of them are resident (H 2048: 52 VGPRs,
    // 8 waves per SIMD, 11.7 -> 10.8 us at 2048 tokens); the chains form keeps
    // four (the two-pass build measured slower at H 4096, 9.4 -> 12.8 us)
    const int np = (H + RO_THREADS * 8 - 1) / (RO_THREADS * 8);
    if (np > RO_MAXPASS) return hipErrorInvalidValue;
    auto go = [&](auto kern) -> hipError_t {
        const size_t lds = route_lds_bytes(H);
        hipError_t e = allow_lds((const void *)kern, lds);
        if (e != hipSuccess) return e;
        TG_LAUNCH(kern, dim3(T), dim3(RO_THREADS), lds, st, raw, chains, T, x, gn, E, H, k, eps, idx, w, xq, xd, xs,
                  ecnt, ent_cap, G);
        return hipGetLastError();
    };
    if (chains) return go(k_route_q8<true, RO_MAXPASS>);
    if (np == 1) return go(k_route_q8<false, 1>);
    if (np == 2) return go(k_route_q8<false, 2>);
    return go(k_route_q8<false, RO_MAXPASS>);
}

bool route_groups_on() {
    const char *v = getenv("TG_ROUTE_GROUP");
    return !(v && v[0] == '0');
}

bool route_chains_usable(int T, int E, int H) { return T < 128 && route_chains_ok(E, H); }

hipError_t launch_route_chains(const float *Wr, const float *x, int T, int E, int H, float *chains, hipStream_t st) {
    if (!route_chains_usable(T, E, H)) return hipErrorInvalidValue;
    if (T <= 64)
        TG_LAUNCH(k_route_chains<16>, dim3(H / RG, cdiv((size_t)T, 16)), dim3(RC_THREADS), 0, st, Wr, x, T, E, H,
                  chains);
    else
        TG_LAUNCH(k_route_chains<32>, dim3(H / RG, cdiv((size_t)T, 32)), dim3(RC_THREADS), 0, st, Wr, x, T, E, H,
                  chains);
    return hipGetLastError();
}

int group_chunk_gateup(const Shape &s) { return gu_chunk(s.nbH); }
int group_chunk_down(const Shape &s) { return dn_chunk(s.nbI, s.I); }

int group_work_max(const Shape &s, int n, int ch) { return s.E + (n + ch - 1) / ch; }

int group_work_max(const Shape &s, int n) {
    const int ch = gu_chunk(s.nbH) < dn_chunk(s.nbI, s.I) ? gu_chunk(s.nbH) : dn_chunk(s.nbI, s.I);
    return group_work_max(s, n, ch);
}

template <bool SORT>
static hipError_t group_go(const int32_t *idx, int n, int E, int ch, int chd, int wmax, int32_t *counts,
                           int32_t *offsets, int32_t *entries, int32_t *work, int32_t *work_n, int32_t *rdy,
                           hipStream_t st) {
    const size_t lds = n <= GR_LDS_ENTRIES ? 4 * (size_t)n : 0;
    hipError_t e = allow_lds((const void *)k_group<SORT>, lds);
    if (e != hipSuccess) return e;
    TG_LAUNCH(k_group<SORT>, dim3(1), dim3(GR_THREADS), lds, st, idx, n, E, ch, chd, wmax, counts, offsets, entries,
              work, work_n, nullptr, 0, rdy);
    return hipGetLastError();
}

hipError_t launch_group(const Shape &s, const int32_t *idx, int n, int32_t *counts, int32_t *offsets,
                        int32_t *entries, int32_t *work, int32_t *work_n, hipStream_t st) {
    return group_go<false>(idx, n, s.E, gu_chunk(s.nbH), dn_chunk(s.nbI, s.I), group_work_max(s, n), counts,
                           offsets, entries, work, work_n, nullptr, st);
}

hipError_t launch_group_placed(const Shape &s, int n, int ch, int cap, int32_t *ecnt, int32_t *counts,
                               int32_t *offsets, int32_t *work, int32_t *work_n, int32_t *rdy, hipStream_t st) {
    const int wmax = group_work_max(s, n, ch);
    if (ch > 32)  // items of several M-tiles: largest first
        TG_LAUNCH((k_group<true, true>), dim3(1), dim3(GR_THREADS), 0, st, nullptr, n, s.E, ch, ch, wmax, counts,
                  offsets, nullptr, work, work_n, ecnt, cap, rdy);
    else
        TG_LAUNCH((k_group<false, true>), dim3(1), dim3(GR_THREADS), 0, st, nullptr, n, s.E, ch, ch, wmax, counts,
                  offsets, nullptr, work, work_n, ecnt, cap, rdy);
    return hipGetLastError();
}

bool place_par_on() {
    const char *v = getenv("TG_GROUP_PAR");
    return !(v && v[0] == '0');
}

hipError_t launch_place(const int32_t *idx, int n, int E, int cap, int32_t *ecnt, int32_t *ent_cap,
                        const RouteGroup &G, hipStream_t st) {
    if (n <= 0 || E > PL_THREADS || E > MAX_E || cap <= 0 || !G.arrive || G.ch <= 0 || G.wmax <= 0 || !G.counts ||
        !G.offsets || !G.work || !G.work_n)
        return hipErrorInvalidValue;
    const unsigned nb = (unsigned)((n + PL_THREADS * PL_PER - 1) / (PL_THREADS * PL_PER));
    TG_LAUNCH(k_place, dim3(nb), dim3(PL_THREADS), 0, st, idx, n, E, cap, ecnt, ent_cap, G);
    return hipGetLastError();
}

hipError_t launch_group_chunked(const Shape &s, const int32_t *idx, int n, int ch, int32_t *counts,
                                int32_t *offsets, int32_t *entries, int32_t *work, int32_t *work_n, int32_t *rdy,
                                hipStream_t st) {
    // items of several M-tiles: largest first (one-tile items are all alike)
    if (ch > 32)
        return group_go<true>(idx, n, s.E, ch, ch, group_work_max(s, n, ch), counts, offsets, entries, work, work_n,
                              rdy, st);
    return group_go<false>(idx, n, s.E, ch, ch, group_work_max(s, n, ch), counts, offsets, entries, work, work_n,
                           rdy, st);
}

template <int NT, int UNR>
static hipError_t gug_go(const uint8_t *layer_pl, const Shape &s, int wmax, const int32_t *work,
                         const int32_t *work_n, const int32_t *entries, const int8_t *xq, const float *xd,
                         const int *xs, int8_t *hq, float *hd, int *hs, hipStream_t st) {
    size_t lds = gu_grouped_lds(s.nbH);
    hipError_t e = allow_lds((const void *)k_gateup_grouped<NT, UNR>, lds);
    if (e != hipSuccess) return e;
    TG_LAUNCH((k_gateup_grouped<NT, UNR>), dim3(s.nbI, wmax), dim3(NT), lds, st, layer_pl, s, work,
                       work_n, entries, xq, xd, xs, hq, hd, hs);
    return hipGetLastError();
}

hipError_t launch_gateup_grouped(const uint8_t *layer_pl, const Shape &s, int n, const int32_t *work,
                                 const int32_t *work_n, const int32_t *entries, const int8_t *xq, const float *xd,
                                 const int *xs, int8_t *hq, float *hd, int *hs, hipStream_t st) {
    if (!grouped_shape_ok(s)) return hipErrorInvalidValue;
    const int wmax = group_work_max(s, n);
    const int per = (int)cdiv((size_t)64 * s.nbH, 256);
    if (per <= 4) return gug_go<256, 4>(layer_pl, s, wmax, work, work_n, entries, xq, xd, xs, hq, hd, hs, st);
    if (per <= 8) return gug_go<256, 8>(layer_pl, s, wmax, work, work_n, entries, xq, xd, xs, hq, hd, hs, st);
    if (per <= 16) return gug_go<256, 16>(layer_pl, s, wmax, work, work_n, entries, xq, xd, xs, hq, hd, hs, st);
    return gug_go<512, 16>(layer_pl, s, wmax, work, work_n, entries, xq, xd, xs, hq, hd, hs, st);
}

template <int UNR>
static hipError_t dng_go(const uint8_t *layer_pl, const Shape &s, int wmax, const int32_t *work,
                         const int32_t *work_n, const int32_t *entries, const int8_t *hq, const float *hd,
                         const int *hs, float *D, hipStream_t st) {
    size_t lds = dn_grouped_lds(s.nbI, s.I);
    hipError_t e = allow_lds((const void *)k_down_grouped<UNR>, lds);
    if (e != hipSuccess) return e;
    TG_LAUNCH(k_down_grouped<UNR>, dim3(s.H / 32, wmax), dim3(RO_THREADS), lds, st, layer_pl, s,
                       work + 3 * (size_t)wmax, work_n, entries, hq, hd, hs, D);
    return hipGetLastError();
}

hipError_t launch_down_grouped(const uint8_t *layer_pl, const Shape &s, int n, const int32_t *work,
                               const int32_t *work_n, const int32_t *entries, const int8_t *hq, const float *hd,
                               const int *hs, float *D, hipStream_t st) {
    if (!grouped_shape_ok(s)) return hipErrorInvalidValue;
    const int wmax = group_work_max(s, n);
    const int per = (int)cdiv((size_t)32 * s.nbI, RO_THREADS);
    if (per <= 2) return dng_go<2>(layer_pl, s, wmax, work, work_n, entries, hq, hd, hs, D, st);
    if (per <= 4) return dng_go<4>(layer_pl, s, wmax, work, work_n, entries, hq, hd, hs, D, st);
    if (per <= 8) return dng_go<8>(layer_pl, s, wmax, work, work_n, entries, hq, hd, hs, D, st);
    return dng_go<16>(layer_pl, s, wmax, work, work_n, entries, hq, hd, hs, D, st);
}

hipError_t launch_combine(const float *D, const float *w, int T, int H, int k, const float *resid, float *out,
                          hipStream_t st) {
    const bool vec = H % 4 == 0 && k <= MAX_K && ((uintptr_t)out & 15) == 0 && ((uintptr_t)resid & 15) == 0 &&
                     ((uintptr_t)D & 15) == 0;
    if (vec)
        TG_LAUNCH(k_combine, dim3(cdiv((size_t)H / 4, 256), T), dim3(256), 0, st, D, w, H, k, resid, out);
    else
        TG_LAUNCH(k_combine1, dim3(cdiv((size_t)H, 256), T), dim3(256), 0, st, D, w, H, k, resid, out);
    return hipGetLastError();
}

}  // namespace tg
