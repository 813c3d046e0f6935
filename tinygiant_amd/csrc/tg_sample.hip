// tg_sample.hip -- temperature / top-p token sampling over a vocabulary of
// logits on the GPU (tinygiant/engine.py:348-357; greedy, :358-359, is the
// argmax of tg_legacy.hip).
//
// The reference samples in numpy:
//   probs = exp((logits - max(logits)) / T);  probs /= sum(probs)
//   order = argsort(probs) descending;  cs = cumsum(probs[order])
//   cutoff = searchsorted(cs, top_p) + 1;  candidates = order[:cutoff]
//   cp = probs[candidates];  cp /= sum(cp);  token = choice(candidates, p=cp)
// where RandomState.choice widens cp to float64, forms cdf = cumsum(cp) /
// cdf[-1], draws one uniform u and takes the first candidate whose cdf value
// exceeds u.  This file computes the same token from the same u, step by
// step in the same arithmetic:
//   z = (l - m) / T in fp32 (correctly rounded division);
//   p = exp(z) as the fp32 rounding of a float64 exp.  numpy's own float32 exp
//       is within 2 ulp of that and differs between CPUs; this build fixes
//       the correctly rounded value;
//   S = np.sum's order: 8192-value buffers added one after another from 0,
//       each buffer by numpy's pairwise recursion (halves rounded down to a
//       multiple of 8 until 128 or fewer values, those by 8 interleaved
//       accumulators combined as ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)) and the
//       last n % 8 values added in order; fewer than 8 values in order from 0);
//   q = p / S;  the fp32 running sum of q in descending order, compared in
//       double with top_p (searchsorted widens the float32 sums);
//   the candidates' sum in np.sum's order, cp = q / that sum, the float64
//       running sum of cp, each value divided by the last, first one > u.
// Ties in q are ordered by ascending token id (numpy's default argsort does
// not fix an order for ties).
//
// Launches of one call (one host synchronisation at the end):
//   k_smp_max     per-block max of the logits and a non-finite flag; clears
//                 the histogram
//   k_smp_exp     p
//   k_smp_chunks  one wave per 8192-value buffer: its pairwise sum
//   k_smp_norm    S from the buffer sums; q = p / S; a histogram of q's top
//                 12 bits with counts and exact mass (units of 2^-40)
//   k_smp_final   the fewest top buckets whose mass provably carries the fp32
//                 running sum past top_p (they hold the candidates); when
//                 they hold at most 8192 elements, their keys (descending q,
//                 ascending id) gathered into LDS, sorted by a bitonic network
//                 8 keys per thread, and the scans by one wave
// More candidates (flat distributions, top_p near 1): the host then gathers
// the keys in global memory (k_smp_compact), sorts them (8192-key tiles in
// registers and LDS, longer steps one launch each), and k_smp_unpack,
// k_smp_cut, k_smp_chunks and k_smp_draw finish.
#include <algorithm>

#include "tg_device.h"
#include "tg_internal.h"

namespace tg {

constexpr int SMP_T = 256;
constexpr int PW_LEVELS = 8;   // depth of numpy's pairwise tree over <= 8192 values is 7
constexpr int BT_TILE = 8192;  // bitonic keys per LDS tile (64 KiB)

TG_DEV uint32_t smp_bucket(float q) {
    const uint32_t b = __float_as_uint(q) >> SMP_BUCKET_SHIFT;
    return b < (uint32_t)SMP_BUCKETS ? b : (uint32_t)SMP_BUCKETS - 1;  // NaN with the sign bit
}
// q in [0, 1] in units of 2^-40, rounded down (exact: a power-of-two scale)
TG_DEV unsigned long long smp_mass(float q) {
    return (q >= 0.0f && q <= 1.0f) ? (unsigned long long)(q * 0x1p40f) : 0ull;
}
// ascending key order = descending q, then ascending id
TG_DEV unsigned long long smp_key(float q, uint32_t id) {
    return ((unsigned long long)(0x7FFFFFFFu - (__float_as_uint(q) & 0x7FFFFFFFu)) << 32) | id;
}
TG_DEV float smp_key_q(unsigned long long k) { return __uint_as_float(0x7FFFFFFFu - (uint32_t)(k >> 32)); }

TG_DEV float rdl(float v, int i) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i)); }
TG_DEV double rdl(double v, int i) {
    const unsigned long long b = __double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, i);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), i);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// ------------------------------------------------ numpy's pairwise sum
// Base case of numpy's pairwise summation, n <= 128 values v[0..n).
TG_DEV float pw_leaf(const float *v, int n) {
    if (n < 8) {
        float r = 0.0f;
        for (int i = 0; i < n; i++) r = r + v[i];
        return r;
    }
    float r0 = v[0], r1 = v[1], r2 = v[2], r3 = v[3], r4 = v[4], r5 = v[5], r6 = v[6], r7 = v[7];
    const int main = n & ~7;
    for (int i = 8; i < main; i += 8) {
        r0 = r0 + v[i]; r1 = r1 + v[i + 1]; r2 = r2 + v[i + 2]; r3 = r3 + v[i + 3];
        r4 = r4 + v[i + 4]; r5 = r5 + v[i + 5]; r6 = r6 + v[i + 6]; r7 = r7 + v[i + 7];
    }
    float res = ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7));
    for (int i = main; i < n; i++) res = res + v[i];
    return res;
}

// The recursion's nodes level by level (at most 64 per level for n <= 8192):
// node (start, len) splits into len/2 rounded down to a multiple of 8 and
// the rest while len > 128.  ch = index of the left child in the next level,
// -1 for a leaf.
struct PwTree {
    short st[PW_LEVELS][WAVE], ln[PW_LEVELS][WAVE], ch[PW_LEVELS][WAVE];
    float v[PW_LEVELS][WAVE];
};

// numpy's pairwise sum of v[0..n), 1 <= n <= 8192, by one whole wave (every
// lane returns it).  Leaves are summed one per lane, inner nodes level by
// level from the bottom, each as left + right.
TG_DEV float wave_pw_sum(const float *v, int n, PwTree &t) {
    const int lane = __lane_id();
    int cnt[PW_LEVELS];
    if (lane == 0) { t.st[0][0] = 0; t.ln[0][0] = (short)n; }
    wave_lds_sync();
    int c = 1;
#pragma unroll
    for (int d = 0; d < PW_LEVELS; d++) {
        cnt[d] = c;
        const bool have = lane < c;
        const int s0 = have ? t.st[d][lane] : 0, l0 = have ? t.ln[d][lane] : 0;
        const bool split = have && l0 > 128 && d + 1 < PW_LEVELS;
        const uint64_t m = __ballot(split);
        const int r = __popcll(m & ((1ull << lane) - 1));
        if (split) {
            const int n2 = (l0 >> 1) & ~7;
            t.st[d + 1][2 * r] = (short)s0;
            t.ln[d + 1][2 * r] = (short)n2;
            t.st[d + 1][2 * r + 1] = (short)(s0 + n2);
            t.ln[d + 1][2 * r + 1] = (short)(l0 - n2);
        }
        if (have) t.ch[d][lane] = (short)(split ? 2 * r : -1);
        c = 2 * __popcll(m);
        wave_lds_sync();
    }
#pragma unroll
    for (int d = PW_LEVELS - 1; d >= 0; d--) {
        if (lane < cnt[d]) {
            const int ch = t.ch[d][lane];
            const int dn = d + 1 < PW_LEVELS ? d + 1 : d;  // children exist only above the last level
            const float val = ch < 0 ? pw_leaf(v + t.st[d][lane], t.ln[d][lane])
                                     : t.v[dn][ch] + t.v[dn][ch + 1];
            t.v[d][lane] = val;
        }
        wave_lds_sync();
    }
    return t.v[0][0];
}

// ------------------------------------------------ one-wave ordered scans
// First k in [0, n) whose fp32 running sum s_k = s_{k-1} + v[k] (s_{-1} = 0)
// satisfies (double)s_k >= top_p, or -1.  The wave forms the sums in order
// (each value read from its lane), 64 per step; the sums only grow, so a
// step whose last sum stays below top_p holds no crossing, and the step that
// crosses is formed again keeping each lane's own sum.
TG_DEV int wave_cut(const float *v, int n, double top_p) {
    constexpr int B = 8;  // values per lane per batch; the next batch is loaded while one is summed
    const int lane = __lane_id();
    float run = 0.0f;
    float x[B], xn[B];
#pragma unroll
    for (int r = 0; r < B; r++) x[r] = r * WAVE + lane < n ? v[r * WAVE + lane] : 0.0f;
    for (int b = 0; b < n; b += B * WAVE) {
#pragma unroll
        for (int r = 0; r < B; r++) {
            const int i = b + (B + r) * WAVE + lane;
            xn[r] = i < n ? v[i] : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < B; r++) {
            const float start = run;
#pragma unroll
            for (int i = 0; i < WAVE; i++) run = run + rdl(x[r], i);
            if ((double)run >= top_p) {
                float s = start, mine = 0.0f;
#pragma unroll
                for (int i = 0; i < WAVE; i++) {
                    s = s + rdl(x[r], i);
                    mine = lane == i ? s : mine;
                }
                const int base = b + r * WAVE;
                const uint64_t hit = __ballot(base + lane < n && (double)mine >= top_p);
                return base + __ffsll((long long)hit) - 1;
            }
        }
#pragma unroll
        for (int r = 0; r < B; r++) x[r] = xn[r];
    }
    return -1;
}

// The float64 running sum of (double)(v[k] / s2) over k < n: its last value
// (cdf[-1] of RandomState.choice).
TG_DEV double wave_total(const float *v, int n, float s2) {
    const int lane = __lane_id();
    double run = 0.0;
    for (int b = 0; b < n; b += WAVE) {
        const double x = b + lane < n ? (double)(v[b + lane] / s2) : 0.0;
#pragma unroll
        for (int i = 0; i < WAVE; i++) run = run + rdl(x, i);
    }
    return run;
}

// First k whose float64 running sum divided by tot exceeds u
// (cdf.searchsorted(u, side='right')); n - 1 if none (u < 1 never gets there).
TG_DEV int wave_draw(const float *v, int n, float s2, double tot, double u) {
    const int lane = __lane_id();
    double run = 0.0;
    for (int b = 0; b < n; b += WAVE) {
        const double x = b + lane < n ? (double)(v[b + lane] / s2) : 0.0;
        const double start = run;
#pragma unroll
        for (int i = 0; i < WAVE; i++) run = run + rdl(x, i);
        if (run / tot > u) {
            double r = start, mine = 0.0;
#pragma unroll
            for (int i = 0; i < WAVE; i++) {
                r = r + rdl(x, i);
                mine = lane == i ? r : mine;
            }
            const uint64_t hit = __ballot(b + lane < n && mine / tot > u);
            return b + __ffsll((long long)hit) - 1;
        }
    }
    return n - 1;
}

// The same draw when every (double)(v[k] / s2) is >= 2^-29: each is then a
// multiple of 2^-52 (24 significant bits), every running sum a multiple of
// 2^-52 below 2, so the float64 running sums are exact and equal the integer
// prefix sums in units of 2^-52, formed here in parallel.
TG_DEV int wave_draw_exact(const float *v, int n, float s2, double u) {
    const int lane = __lane_id();
    unsigned long long tot = 0;
    for (int b = 0; b < n; b += WAVE) {
        unsigned long long x = b + lane < n ? (unsigned long long)((double)(v[b + lane] / s2) * 0x1p52) : 0ull;
        for (int s = WAVE / 2; s >= 1; s >>= 1) x += __shfl_xor(x, s, WAVE);
        tot += x;
    }
    const double dt = (double)tot * 0x1p-52;
    unsigned long long run = 0;
    for (int b = 0; b < n; b += WAVE) {
        unsigned long long x = b + lane < n ? (unsigned long long)((double)(v[b + lane] / s2) * 0x1p52) : 0ull;
        for (int s = 1; s < WAVE; s <<= 1) {  // inclusive scan over the wave
            const unsigned long long o = __shfl_up(x, s, WAVE);
            if (lane >= s) x += o;
        }
        const double cdf = (double)(run + x) * 0x1p-52;
        const uint64_t hit = __ballot(b + lane < n && cdf / dt > u);
        if (hit) return b + __ffsll((long long)hit) - 1;
        run += __shfl(x, WAVE - 1, WAVE);
    }
    return n - 1;
}

// np.sum of v[0..n) as buffers of 8192 added from 0, by one wave
TG_DEV float wave_np_sum(const float *v, int n, PwTree &t) {
    float s = 0.0f;
    for (int c0 = 0; c0 < n; c0 += NP_BUFSIZE) s = s + wave_pw_sum(v + c0, min(NP_BUFSIZE, n - c0), t);
    return s;
}

// The position drawn among the first cut values (cp = v / s2, descending).
TG_DEV int wave_pick(const float *v, int cut, float s2, double u) {
    if (v[cut - 1] / s2 >= 0x1p-29f) return wave_draw_exact(v, cut, s2, u);
    return wave_draw(v, cut, s2, wave_total(v, cut, s2), u);
}

// The candidates' draw from their q in descending order (v[0..n)): writes
// cut and the token drawn.
TG_DEV void wave_finish(const float *v, int n, int V, double top_p, double u, PwTree &t, SmpCtl *ctl,
                        const uint32_t *ids) {
    int cut = wave_cut(v, n, top_p);
    if (cut < 0) {
        if (n != V) {  // the selection bound guarantees a crossing inside a strict prefix
            if (__lane_id() == 0) ctl->status = SMP_ST_BOUND;
            return;
        }
        cut = V;  // searchsorted past the end: every token is a candidate
    } else {
        cut += 1;
    }
    const float s2 = wave_np_sum(v, cut, t);
    const int pos = wave_pick(v, cut, s2, u);
    if (__lane_id() == 0) {
        ctl->cut = cut;
        ctl->token = (int)ids[pos];
        ctl->status = SMP_ST_OK;
    }
}

// ------------------------------------------------ kernels
__global__ __launch_bounds__(SMP_T) void k_smp_max(const float *__restrict__ l, int V, float *__restrict__ pmax,
                                                   int *__restrict__ pbad, uint32_t *__restrict__ hcnt,
                                                   unsigned long long *__restrict__ hmass, SmpCtl *ctl) {
    const int tid = threadIdx.x, gt = blockIdx.x * SMP_T + tid, gn = gridDim.x * SMP_T;
    for (int b = gt; b < SMP_BUCKETS; b += gn) { hcnt[b] = 0; hmass[b] = 0; }
    if (gt == 0) { ctl->n = 0; ctl->done = 0; ctl->large = 0; ctl->status = SMP_ST_PENDING; ctl->token = -1; ctl->cut = 0; }
    float m = -INFINITY;
    int bad = 0;
    for (int i = gt; i < V; i += gn) {
        const float x = l[i];
        bad |= (x != x) | (x == INFINITY);
        m = fmaxf(m, x);
    }
    for (int s = WAVE / 2; s >= 1; s >>= 1) {
        m = fmaxf(m, __shfl_xor(m, s, WAVE));
        bad |= __shfl_xor(bad, s, WAVE);
    }
    __shared__ float sm[SMP_T / WAVE];
    __shared__ int sb[SMP_T / WAVE];
    if ((tid & (WAVE - 1)) == 0) { sm[tid / WAVE] = m; sb[tid / WAVE] = bad; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < SMP_T / WAVE; w++) { m = fmaxf(m, sm[w]); bad |= sb[w]; }
        pmax[blockIdx.x] = m;
        pbad[blockIdx.x] = bad;
    }
}

__global__ __launch_bounds__(SMP_T) void k_smp_exp(const float *__restrict__ l, int V, const float *__restrict__ pmax,
                                                   const int *__restrict__ pbad, int nb, float T,
                                                   float *__restrict__ p, SmpCtl *ctl) {
    __shared__ float s_m;
    const int tid = threadIdx.x;
    if (tid < WAVE) {
        float m = -INFINITY;
        int bad = 0;
        for (int b = tid; b < nb; b += WAVE) { m = fmaxf(m, pmax[b]); bad |= pbad[b]; }
        for (int s = WAVE / 2; s >= 1; s >>= 1) {
            m = fmaxf(m, __shfl_xor(m, s, WAVE));
            bad |= __shfl_xor(bad, s, WAVE);
        }
        if (tid == 0) {
            s_m = m;
            if (blockIdx.x == 0) { ctl->m = m; ctl->bad = bad | (m == -INFINITY); }
        }
    }
    __syncthreads();
    const float m = s_m;
    for (int i = blockIdx.x * SMP_T + tid; i < V; i += gridDim.x * SMP_T) {
        const float z = (l[i] - m) / T;
        p[i] = (float)exp((double)z);
    }
}

// One wave per 8192-value buffer of v[0..n): its pairwise sum.  n is the
// argument, or, when n_from_ctl, the candidate count ctl->cut.
__global__ __launch_bounds__(WAVE) void k_smp_chunks(const float *__restrict__ v, int n, int n_from_ctl,
                                                     const SmpCtl *ctl, float *__restrict__ sums) {
    __shared__ PwTree t;
    if (n_from_ctl) {
        if (ctl->status != SMP_ST_PENDING) return;
        n = ctl->cut;
    }
    const int c0 = blockIdx.x * NP_BUFSIZE;
    if (c0 >= n) return;
    const float s = wave_pw_sum(v + c0, min(NP_BUFSIZE, n - c0), t);
    if (threadIdx.x == 0) sums[blockIdx.x] = s;
}

// The candidates lie in the top buckets: with C elements and exact mass M
// (2^-40 units, rounded down per element) in buckets >= b, the fp32 running
// sum over those elements in descending order ends at or above
// M 2^-40 - C 2^-24 (each addition rounds by at most half an ulp of a sum
// below 2), so M 2^-40 >= top_p + C 2^-24 puts the crossing inside them.
// The largest such b is taken; none (top_p near or above 1, or NaN) = all.
// A block of NT threads; the histogram is read at device scope (other
// blocks' atomics).  Leaves bstar and C in ctl.
template <int NT>
TG_DEV void smp_select(const uint32_t *hcnt, const unsigned long long *hmass, int V, double top_p, SmpCtl *ctl) {
    constexpr int PER = SMP_BUCKETS / NT;
    __shared__ uint32_t wc[NT / WAVE];
    __shared__ unsigned long long wm[NT / WAVE];
    __shared__ int s_best;
    __shared__ uint32_t s_C;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid / WAVE;
    // descending position d = PER tid + k holds bucket SMP_BUCKETS - 1 - d
    uint32_t c[PER];
    unsigned long long ms[PER];
    uint32_t tc = 0;
    unsigned long long tm = 0;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int b = SMP_BUCKETS - 1 - (PER * tid + k);
        c[k] = __hip_atomic_load(hcnt + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ms[k] = __hip_atomic_load(hmass + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        tc += c[k];
        tm += ms[k];
    }
    uint32_t ic = tc;  // inclusive scan of the thread totals over the wave, then over waves
    unsigned long long im = tm;
    for (int s = 1; s < WAVE; s <<= 1) {
        const uint32_t oc = __shfl_up(ic, s, WAVE);
        const unsigned long long om = __shfl_up(im, s, WAVE);
        if (lane >= s) { ic += oc; im += om; }
    }
    if (lane == WAVE - 1) { wc[w] = ic; wm[w] = im; }
    if (tid == 0) { s_best = INT_MAX; s_C = (uint32_t)V; }
    __syncthreads();
    uint32_t cc = ic - tc;
    unsigned long long cm = im - tm;
    for (int j = 0; j < w; j++) { cc += wc[j]; cm += wm[j]; }
    int best = INT_MAX;
    uint32_t bestC = 0;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        cc += c[k];
        cm += ms[k];
        const double need = (top_p + (double)cc * 0x1p-24) * 0x1p40 + 1024.0;
        if (best == INT_MAX && cc >= 1 && (double)cm >= need) { best = PER * tid + k; bestC = cc; }
    }
    atomicMin(&s_best, best);
    __syncthreads();
    if (best != INT_MAX && best == s_best) s_C = bestC;
    __syncthreads();
    if (tid == 0) {
        const int d = s_best;
        ctl->bstar = d == INT_MAX ? 0 : SMP_BUCKETS - 1 - d;
        ctl->C = d == INT_MAX ? (uint32_t)V : s_C;
    }
}

__global__ __launch_bounds__(SMP_T) void k_smp_norm(const float *__restrict__ p, int V,
                                                    const float *__restrict__ sums, int nchunks, double top_p,
                                                    SmpCtl *ctl, float *__restrict__ q, uint32_t *hcnt,
                                                    unsigned long long *hmass) {
    __shared__ uint32_t lc[SMP_BUCKETS];
    __shared__ unsigned long long lm[SMP_BUCKETS];
    __shared__ float s_S;
    __shared__ int s_last;
    const int tid = threadIdx.x;
    for (int b = tid; b < SMP_BUCKETS; b += SMP_T) { lc[b] = 0; lm[b] = 0; }
    if (tid == 0) {
        float S = 0.0f;
        for (int c = 0; c < nchunks; c++) S = S + sums[c];
        s_S = S;
        if (blockIdx.x == 0) ctl->S = S;
    }
    __syncthreads();
    const float S = s_S;
    for (int i = blockIdx.x * SMP_T + tid; i < V; i += gridDim.x * SMP_T) {
        const float v = p[i] / S;
        q[i] = v;
        const uint32_t b = smp_bucket(v);
        atomicAdd(&lc[b], 1u);
        atomicAdd(&lm[b], smp_mass(v));
    }
    __syncthreads();
    for (int b = tid; b < SMP_BUCKETS; b += SMP_T)
        if (lc[b]) {
            atomicAdd(&hcnt[b], lc[b]);
            atomicAdd(&hmass[b], lm[b]);
        }
    // the last block to finish picks the candidate buckets
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = atomicAdd(&ctl->done, 1u) == gridDim.x - 1;
    __syncthreads();
    if (s_last) {
        __threadfence();
        smp_select<SMP_T>(hcnt, hmass, V, top_p, ctl);
    }
}

// Bitonic network, 8 keys per thread: thread t holds keys 8t .. 8t+7 of a
// run whose first key is key g0 of the whole network (g0 a multiple of 8192;
// the direction of stage kk at key i is ascending when (i & kk) == 0).  One
// step (kk, j): j < 8 in registers, 8 <= j < 512 with lane t ^ (j / 8) of the
// same wave, larger through LDS (x, 8 keys per thread).  Every thread of the
// block calls it; threads with 8t >= n hold no keys (n a power of two >= 8).
template <int J>
TG_DEV void bt_reg_step(unsigned long long (&k)[8], uint32_t g, int kk) {
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const int l = r ^ J;
        if (l > r) {
            const bool asc = ((g + (uint32_t)r) & (uint32_t)kk) == 0;
            const unsigned long long a = k[r], b = k[l];
            if ((a > b) == asc) { k[r] = b; k[l] = a; }
        }
    }
}

TG_DEV unsigned long long shfl_xor_u64(unsigned long long v, int m) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m, WAVE);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m, WAVE);
    return ((unsigned long long)hi << 32) | lo;
}

TG_DEV unsigned long long bt_pick(unsigned long long a, unsigned long long o, bool keep_min) {
    return keep_min ? (a < o ? a : o) : (a > o ? a : o);
}

TG_DEV void bt_step(unsigned long long (&k)[8], int n, uint32_t g0, int kk, int j, unsigned long long *x) {
    const int t = threadIdx.x;
    const bool act = (t << 3) < n;
    const uint32_t g = g0 + ((uint32_t)t << 3);
    if (j >= 512) {
        if (act) {
#pragma unroll
            for (int r = 0; r < 8; r++) x[(t << 3) + r] = k[r];
        }
        __syncthreads();
        if (act) {
#pragma unroll
            for (int r = 0; r < 8; r++) {
                const int i = (t << 3) + r;
                const bool keep_min = (((g + (uint32_t)r) & (uint32_t)kk) == 0) == ((i & j) == 0);
                k[r] = bt_pick(k[r], x[i ^ j], keep_min);
            }
        }
        __syncthreads();
    } else if (j >= 8) {
        const int m = j >> 3;  // partner lane t ^ m, in the same wave (m < 64)
#pragma unroll
        for (int r = 0; r < 8; r++) {
            const unsigned long long o = shfl_xor_u64(k[r], m);
            const bool keep_min = (((g + (uint32_t)r) & (uint32_t)kk) == 0) == ((t & m) == 0);
            k[r] = bt_pick(k[r], o, keep_min);
        }
    } else if (j == 4) {
        bt_reg_step<4>(k, g, kk);
    } else if (j == 2) {
        bt_reg_step<2>(k, g, kk);
    } else {
        bt_reg_step<1>(k, g, kk);
    }
}

// Ascending sort of n keys (8 <= n <= 8192, a power of two) held 8 per thread.
TG_DEV void bitonic_regs(unsigned long long (&k)[8], int n, unsigned long long *x) {
    for (int kk = 2; kk <= n; kk <<= 1)
        for (int j = kk >> 1; j > 0; j >>= 1) bt_step(k, n, 0, kk, j, x);
}

// The last launch of a call: at most 8192 candidates (keys[0..C) from
// k_smp_compact) sorted in registers and LDS, then the scans by wave 0.
// More candidates: ctl->large for the host.
__global__ __launch_bounds__(1024) void k_smp_final(const unsigned long long *__restrict__ keys, int V,
                                                    double top_p, double u, SmpCtl *ctl) {
    extern __shared__ __align__(16) uint8_t smem[];
    unsigned long long *sk = reinterpret_cast<unsigned long long *>(smem);
    PwTree &t = *reinterpret_cast<PwTree *>(smem + sizeof(unsigned long long) * SMP_SMALL);
    const int tid = threadIdx.x;
    if (ctl->bad) {
        if (tid == 0) ctl->status = SMP_ST_INPUT;
        return;
    }
    const uint32_t C = ctl->C;
    if (C > (uint32_t)SMP_SMALL) {
        if (tid == 0) ctl->large = 1;
        return;
    }
    int P = 8;
    while (P < (int)C) P <<= 1;
    unsigned long long k[8];
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const int i = (tid << 3) + r;
        k[r] = i < (int)C ? keys[i] : ~0ull;
    }
    bitonic_regs(k, P, sk);
    __syncthreads();
    // sorted keys -> q (first half of the array) and ids (second half)
    float *sq = reinterpret_cast<float *>(smem);
    uint32_t *sid = reinterpret_cast<uint32_t *>(smem) + SMP_SMALL;
#pragma unroll
    for (int r = 0; r < 8; r++) {
        const int i = (tid << 3) + r;
        if (i < (int)C) {
            sq[i] = smp_key_q(k[r]);
            sid[i] = (uint32_t)k[r];
        }
    }
    __syncthreads();
    if (tid < WAVE) wave_finish(sq, (int)C, V, top_p, u, t, ctl, sid);
}

// ------------------------------------------------ more than 8192 candidates
// The candidates' keys (bucket >= ctl->bstar) into keys[0..C): per block a
// count, one global slot range, then the keys.
__global__ __launch_bounds__(SMP_T) void k_smp_compact(const float *__restrict__ q, int V, SmpCtl *ctl,
                                                       unsigned long long *__restrict__ keys) {
    __shared__ uint32_t s_cnt, s_base;
    const uint32_t bstar = (uint32_t)ctl->bstar;
    const int lane = __lane_id();
    if (threadIdx.x == 0) s_cnt = 0;
    __syncthreads();
    for (int i = blockIdx.x * SMP_T + threadIdx.x; i < V; i += gridDim.x * SMP_T)
        if (smp_bucket(q[i]) >= bstar) atomicAdd(&s_cnt, 1u);
    __syncthreads();
    if (threadIdx.x == 0) {
        s_base = atomicAdd(&ctl->n, s_cnt);
        s_cnt = 0;
    }
    __syncthreads();
    for (int i0 = blockIdx.x * SMP_T; i0 < V; i0 += gridDim.x * SMP_T) {
        const int i = i0 + threadIdx.x;
        float v = 0.0f;
        bool take = false;
        if (i < V) {
            v = q[i];
            take = smp_bucket(v) >= bstar;
        }
        const uint64_t m = __ballot(take);
        if (m) {
            const int leader = __ffsll((long long)m) - 1;
            uint32_t base = 0;
            if (lane == leader) base = atomicAdd(&s_cnt, (uint32_t)__popcll(m));
            base = (uint32_t)__shfl((int)base, leader, WAVE);
            if (take) keys[s_base + base + __popcll(m & ((1ull << lane) - 1))] = smp_key(v, (uint32_t)i);
        }
    }
}

__global__ __launch_bounds__(SMP_T) void k_fill_u64(unsigned long long *__restrict__ p, int from, int to,
                                                    unsigned long long v) {
    for (int i = from + blockIdx.x * SMP_T + threadIdx.x; i < to; i += gridDim.x * SMP_T) p[i] = v;
}

// Each 8192-key tile through the stages kk = 2..8192 of the global network,
// or, with kfix, the steps j = 4096..1 of stage kfix.
__global__ __launch_bounds__(1024) void k_bitonic_tile(unsigned long long *__restrict__ keys, int kfix) {
    __shared__ unsigned long long x[BT_TILE];
    const uint32_t g0 = blockIdx.x * BT_TILE;
    unsigned long long k[8];
#pragma unroll
    for (int r = 0; r < 8; r++) k[r] = keys[g0 + (threadIdx.x << 3) + r];
    if (kfix) {
        for (int j = BT_TILE / 2; j > 0; j >>= 1) bt_step(k, BT_TILE, g0, kfix, j, x);
    } else {
        for (int kk = 2; kk <= BT_TILE; kk <<= 1)
            for (int j = kk >> 1; j > 0; j >>= 1) bt_step(k, BT_TILE, g0, kk, j, x);
    }
#pragma unroll
    for (int r = 0; r < 8; r++) keys[g0 + (threadIdx.x << 3) + r] = k[r];
}

// One step (kk, j >= 8192) of the network: one pair per thread.
__global__ __launch_bounds__(SMP_T) void k_bitonic_step(unsigned long long *__restrict__ keys, int j, int k) {
    const uint32_t t = blockIdx.x * SMP_T + threadIdx.x;
    const uint32_t i = ((t / (uint32_t)j) * 2u * (uint32_t)j) + (t % (uint32_t)j), l = i + (uint32_t)j;
    const unsigned long long a = keys[i], b = keys[l];
    const bool asc = (i & (uint32_t)k) == 0;
    if ((a > b) == asc) { keys[i] = b; keys[l] = a; }
}

__global__ __launch_bounds__(SMP_T) void k_smp_unpack(const unsigned long long *__restrict__ keys, int C,
                                                      float *__restrict__ sq, uint32_t *__restrict__ sid) {
    for (int i = blockIdx.x * SMP_T + threadIdx.x; i < C; i += gridDim.x * SMP_T) {
        const unsigned long long k = keys[i];
        sq[i] = smp_key_q(k);
        sid[i] = (uint32_t)k;
    }
}

__global__ __launch_bounds__(WAVE) void k_smp_cut(const float *__restrict__ sq, int C, int V, double top_p,
                                                  SmpCtl *ctl) {
    const int c = wave_cut(sq, C, top_p);
    if (threadIdx.x == 0) {
        if (c >= 0) ctl->cut = c + 1;
        else if (C == V) ctl->cut = V;
        else ctl->status = SMP_ST_BOUND;
    }
}

// The draw over cut candidates in global memory.  When every cp >= 2^-29
// (the exact case of wave_draw_exact) the block's 16 waves take one segment
// each: segment totals, their prefix, then each wave finds its first hit and
// the lowest position wins; otherwise wave 0 alone, in order.
__global__ __launch_bounds__(1024) void k_smp_draw(const float *__restrict__ sq, const uint32_t *__restrict__ sid,
                                                   const float *__restrict__ sums, double u, SmpCtl *ctl) {
    constexpr int NW = 1024 / WAVE;
    __shared__ unsigned long long seg[NW];
    __shared__ int s_pos;
    if (ctl->status != SMP_ST_PENDING) return;
    const int cut = ctl->cut, tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid / WAVE;
    float s2 = 0.0f;
    for (int c = 0; c * NP_BUFSIZE < cut; c++) s2 = s2 + sums[c];
    if (!(sq[cut - 1] / s2 >= 0x1p-29f)) {
        if (tid < WAVE) {
            const int pos = wave_draw(sq, cut, s2, wave_total(sq, cut, s2), u);
            if (tid == 0) {
                ctl->token = (int)sid[pos];
                ctl->status = SMP_ST_OK;
            }
        }
        return;
    }
    const int len = ((cut + NW - 1) / NW + WAVE - 1) / WAVE * WAVE;
    const int lo = min(cut, w * len), hi = min(cut, lo + len);
    auto units = [&](int i) -> unsigned long long {
        return i < hi ? (unsigned long long)((double)(sq[i] / s2) * 0x1p52) : 0ull;
    };
    unsigned long long tot = 0;
    for (int b = lo; b < hi; b += WAVE) {
        unsigned long long x = units(b + lane);
        for (int s = WAVE / 2; s >= 1; s >>= 1) x += __shfl_xor(x, s, WAVE);
        tot += x;
    }
    if (lane == 0) seg[w] = tot;
    if (tid == 0) s_pos = INT_MAX;
    __syncthreads();
    unsigned long long run = 0, all = 0;
    for (int j = 0; j < NW; j++) {
        if (j < w) run += seg[j];
        all += seg[j];
    }
    const double dt = (double)all * 0x1p-52;
    for (int b = lo; b < hi; b += WAVE) {
        unsigned long long x = units(b + lane);
        for (int s = 1; s < WAVE; s <<= 1) {
            const unsigned long long o = __shfl_up(x, s, WAVE);
            if (lane >= s) x += o;
        }
        const double cdf = (double)(run + x) * 0x1p-52;
        const uint64_t hit = __ballot(b + lane < hi && cdf / dt > u);
        if (hit) {
            if (lane == 0) atomicMin(&s_pos, b + __ffsll((long long)hit) - 1);
            break;
        }
        run += __shfl(x, WAVE - 1, WAVE);
    }
    __syncthreads();
    if (tid == 0) {
        const int pos = s_pos == INT_MAX ? cut - 1 : s_pos;
        ctl->token = (int)sid[pos];
        ctl->status = SMP_ST_OK;
    }
}

// ------------------------------------------------ launchers
static unsigned smp_grid(long n, long per) { return (unsigned)std::max<long>(1, std::min<long>(256, (n + per - 1) / per)); }

size_t smp_small_lds() { return sizeof(unsigned long long) * SMP_SMALL + sizeof(PwTree); }

hipError_t launch_sample_main(const SmpBufs &b, const float *logits, int V, float T, double top_p, double u,
                              hipStream_t st) {
    if (V <= 0 || V > SMP_VMAX) return hipErrorInvalidValue;
    const unsigned nb = smp_grid(V, SMP_T * 4);
    const int nchunks = (V + NP_BUFSIZE - 1) / NP_BUFSIZE;
    TG_LAUNCH(k_smp_max, dim3(nb), dim3(SMP_T), 0, st, logits, V, b.pmax, b.pbad, b.hcnt, b.hmass, b.ctl);
    TG_LAUNCH(k_smp_exp, dim3(smp_grid(V, SMP_T * 2)), dim3(SMP_T), 0, st, logits, V, b.pmax, b.pbad, (int)nb, T,
              b.p, b.ctl);
    TG_LAUNCH(k_smp_chunks, dim3(nchunks), dim3(WAVE), 0, st, b.p, V, 0, b.ctl, b.sums);
    TG_LAUNCH(k_smp_norm, dim3(smp_grid(V, SMP_T * 8)), dim3(SMP_T), 0, st, b.p, V, b.sums, nchunks, top_p, b.ctl,
              b.q, b.hcnt, b.hmass);
    TG_LAUNCH(k_smp_compact, dim3(smp_grid(V, SMP_T * 8)), dim3(SMP_T), 0, st, b.q, V, b.ctl, b.keys);
    TG_LAUNCH(k_smp_final, dim3(1), dim3(1024), smp_small_lds(), st, b.keys, V, top_p, u, b.ctl);
    return hipGetLastError();
}

hipError_t launch_sample_large(const SmpBufs &b, int V, int C, double top_p, double u, hipStream_t st) {
    if (C <= SMP_SMALL || C > V || V > SMP_VMAX) return hipErrorInvalidValue;
    int P = BT_TILE;
    while (P < C) P <<= 1;
    TG_LAUNCH(k_fill_u64, dim3(smp_grid(P - C, SMP_T)), dim3(SMP_T), 0, st, b.keys, C, P, ~0ull);
    const int tiles = P / BT_TILE;
    TG_LAUNCH(k_bitonic_tile, dim3(tiles), dim3(1024), 0, st, b.keys, 0);
    for (int k = 2 * BT_TILE; k <= P; k <<= 1) {
        for (int j = k >> 1; j >= BT_TILE; j >>= 1)
            TG_LAUNCH(k_bitonic_step, dim3(P / 2 / SMP_T), dim3(SMP_T), 0, st, b.keys, j, k);
        TG_LAUNCH(k_bitonic_tile, dim3(tiles), dim3(1024), 0, st, b.keys, k);
    }
    const int nchunks = (V + NP_BUFSIZE - 1) / NP_BUFSIZE;
    TG_LAUNCH(k_smp_unpack, dim3(smp_grid(C, SMP_T * 4)), dim3(SMP_T), 0, st, b.keys, C, b.sq, b.sid);
    TG_LAUNCH(k_smp_cut, dim3(1), dim3(WAVE), 0, st, b.sq, C, V, top_p, b.ctl);
    TG_LAUNCH(k_smp_chunks, dim3(nchunks), dim3(WAVE), 0, st, b.sq, 0, 1, b.ctl, b.sums);
    TG_LAUNCH(k_smp_draw, dim3(1), dim3(1024), 0, st, b.sq, b.sid, b.sums, u, b.ctl);
    return hipGetLastError();
}

hipError_t sample_prepare() {
    return hipFuncSetAttribute((const void *)k_smp_final, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)smp_small_lds());
}

}  // namespace tg
