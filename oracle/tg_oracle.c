/*
 * tg_oracle.c -- CPU restatement of TinyGiant's MoE expert hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker).  Loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg; never by the
 * product library.  Build: oracle/Makefile (gcc -O3 -ffp-contract=off).
 *
 * The reference (csrc/libtinygiant.c) is ARM-NEON-only and has no Q4_0/Q8_0
 * kernels; this file restates its algorithm (quantize the activation once,
 * integer block dots, fp32 per-block scaling, SiLU*up, weighted accumulate)
 * for the Q4_0/Q8_0 formats, and restates its Q4_K/Q6_K/f16 functions for
 * the legacy ABI.  Each function names the reference lines it follows and
 * the test in tests/ that pins it.
 *
 * Floating-point order.  Every sum is written out in the exact order the
 * GPU kernels use, with fmaf where the kernels fuse, so that the GPU output
 * is bit-identical to this file's output.  That order is:
 *   row dot      acc = fma(round(S_b * dw_b), dx_b, acc), blocks b = 0..nb-1
 *                (S_b = exact int32 block sum; the same sequential per-block
 *                accumulation as libtinygiant.c:109-167 `total += ...`)
 *   sum of x^2   fma chain inside each group of 32 consecutive elements,
 *                group sums added in ascending order
 *   router       logit = s * (w . x) with w . x in the same grouped order and
 *                s = 1/sqrt(mean(x^2) + eps)
 *   softmax sum  numpy's pairwise float32 sum over the top-k in ascending
 *                logit order (engine.py:232-236)
 *   combine      acc = fma(w_j, down_j, acc) in ascending logit order
 *                (engine.py:240-257, libtinygiant.c:593-594)
 */
#include "tg_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* ------------------------------------------------------------------ */
/* conversions                                                          */
/* ------------------------------------------------------------------ */

/* IEEE binary16 -> binary32, subnormals normalised, e=31 -> inf/NaN with the
 * payload kept.  Follows csrc/libtinygiant.c:24-33.
 * Pinned by tests/test_oracle_formats.py::test_f16_to_f32_exhaustive (all
 * 65,536 codes against numpy) and the reference test constants 0x3400,
 * 0x2C00 (csrc/test_libtinygiant.c:66-67) and 0x2000
 * (tools/nws_fused_bench.c:80). */
float tgo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: shift the mantissa up until the implicit bit appears */
        int e = 1;
        while (!(man & 0x400u)) { man <<= 1; e--; }
        man &= 0x3FFu;
        return u2f(sign | ((uint32_t)(e + 112) << 23) | (man << 13));
    }
    if (exp == 31) return u2f(sign | 0x7F800000u | (man << 13));
    return u2f(sign | ((exp + 112) << 23) | (man << 13));
}

/* Array form (keeps signalling-NaN payloads, which a float return value
 * passed through a host ABI may quiet). */
void tgo_f16_to_f32_n(const uint16_t *h, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = tgo_f16_to_f32(h[i]);
}

/* binary32 -> binary16, round to nearest even, overflow to inf, NaN quieted.
 * This is the rounding of ggml's fp16 store (D1/D2 scale storage) and of the
 * GPU's v_cvt_f16_f32.  Pinned by
 * tests/test_oracle_formats.py::test_f32_to_f16_matches_numpy. */
uint16_t tgo_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {                       /* inf or NaN */
        if (ax == 0x7F800000u) return sign | 0x7C00u;
        return sign | 0x7E00u | (uint16_t)((ax >> 13) & 0x3FFu);
    }
    if (ax >= 0x477FF000u) return sign | 0x7C00u;  /* >= 65520 rounds to inf */
    if (ax >= 0x38800000u) {                       /* normal half */
        uint32_t h = (ax >> 13) - ((127u - 15u) << 10);
        uint32_t rb = ax & 0x1FFFu;
        if (rb > 0x1000u || (rb == 0x1000u && (h & 1u))) h++;
        return sign | (uint16_t)h;
    }
    if (ax < 0x33000000u) return sign;             /* below 2^-25 */
    {                                              /* subnormal half */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;                 /* 14..24 */
        uint32_t h = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return sign | (uint16_t)h;
    }
}

/* ------------------------------------------------------------------ */
/* elementary functions used on the path                                */
/* ------------------------------------------------------------------ */

/* exp(x): Cody-Waite reduction x = n*ln2 + r (ln2 split in a 15-bit head and
 * a tail so n*head is exact), e^r by its degree-7 Taylor polynomial in Horner
 * form with fmaf, scaled by 2^n with ldexpf.  Arguments are clamped to
 * [-87, 88] so every result is a finite normal float.  Used for SiLU
 * (libtinygiant.c:581) and the router softmax (engine.py:234) in place of
 * libm's expf so that host and GPU round identically.
 * Pinned by tests/test_oracle_math.py::test_expf_ulp (<= 2 ulp against the
 * float64 exponential over a dense sweep). */
float tgo_expf(float x) {
    if (x > 88.0f) x = 88.0f;
    if (x < -87.0f) x = -87.0f;
    float n = rintf(x * 1.44269502f);
    float r = fmaf(n, -0.693145751953125f, x);
    r = fmaf(n, -1.42860677e-06f, r);
    float p = 1.98412698e-04f;          /* 1/7! */
    p = fmaf(p, r, 1.38888889e-03f);    /* 1/6! */
    p = fmaf(p, r, 8.33333333e-03f);    /* 1/5! */
    p = fmaf(p, r, 4.16666667e-02f);    /* 1/4! */
    p = fmaf(p, r, 1.66666667e-01f);    /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

/* ln(u) for u in (0, 1], used only by the synthetic-data generator:
 * u = m * 2^e with m in [sqrt(1/2), sqrt(2)), ln m = 2 atanh(s) with
 * s = (m-1)/(m+1), series to s^11.  Pinned by
 * tests/test_oracle_math.py::test_ln_unit (< 4e-7 absolute error). */
float tgo_ln_unit(float u) {
    uint32_t b = f2u(u);
    int e = (int)((b >> 23) & 0xFFu) - 127;
    float m = u2f((b & 0x7FFFFFu) | 0x3F800000u);
    if (m > 1.41421356f) { m = m * 0.5f; e = e + 1; }
    float f = m - 1.0f;
    float s = f / (2.0f + f);
    float z = s * s;
    float p = 0.0909090909f;            /* 1/11 */
    p = fmaf(p, z, 0.111111111f);       /* 1/9 */
    p = fmaf(p, z, 0.142857143f);       /* 1/7 */
    p = fmaf(p, z, 0.2f);
    p = fmaf(p, z, 0.333333333f);
    p = fmaf(p, z, 1.0f);
    float lnm = (2.0f * s) * p;
    return fmaf((float)e, 0.693147182f, lnm);
}

/* cos(2*pi*u) for u in [0, 1): quadrant from 4u, then Taylor series of cos
 * (to theta^14) or sin (to theta^15) on [0, pi/2).  Generator only.  Pinned
 * by tests/test_oracle_math.py::test_cos2pi (< 2e-7 absolute error). */
float tgo_cos2pi(float u) {
    int q = (int)(u * 4.0f);
    if (q > 3) q = 3;
    float r = u - 0.25f * (float)q;
    float t = r * 6.28318531f;
    float z = t * t;
    float c = -1.14707456e-11f;         /* -1/14! */
    c = fmaf(c, z, 2.08767570e-09f);    /* 1/12! */
    c = fmaf(c, z, -2.75573192e-07f);   /* -1/10! */
    c = fmaf(c, z, 2.48015873e-05f);    /* 1/8! */
    c = fmaf(c, z, -1.38888889e-03f);   /* -1/6! */
    c = fmaf(c, z, 4.16666667e-02f);    /* 1/4! */
    c = fmaf(c, z, -0.5f);
    c = fmaf(c, z, 1.0f);
    /* sin t = t + t z P(z), P(z) = -1/3! + z/5! - ... - z^6/15! */
    float s = -7.64716373e-13f;         /* -1/15! */
    s = fmaf(s, z, 1.60590438e-10f);    /* 1/13! */
    s = fmaf(s, z, -2.50521084e-08f);   /* -1/11! */
    s = fmaf(s, z, 2.75573192e-06f);    /* 1/9! */
    s = fmaf(s, z, -1.98412698e-04f);   /* -1/7! */
    s = fmaf(s, z, 8.33333333e-03f);    /* 1/5! */
    s = fmaf(s, z, -1.66666667e-01f);   /* -1/3! */
    s = s * z;
    s = fmaf(s, t, t);
    switch (q) {
    case 0: return c;
    case 1: return -s;
    case 2: return -c;
    default: return s;
    }
}

/* ------------------------------------------------------------------ */
/* synthetic data: SplitMix64 counters + Box-Muller                     */
/* ------------------------------------------------------------------ */

/* SplitMix64 finaliser (Steele, Lea & Flood, OOPSLA 2014). */
uint64_t tgo_splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t tgo_stream_key(uint64_t seed, uint64_t stream) {
    return tgo_splitmix64(seed ^ tgo_splitmix64(stream ^ 0x6A09E667F3BCC909ull));
}

/* One N(0,1) draw per counter: 24-bit u1 in (0,1], 24-bit u2 in [0,1),
 * z = sqrt(-2 ln u1) cos(2 pi u2), all in float32 with the functions above,
 * so that the GPU generator reproduces the bytes exactly. */
float tgo_normal_at(uint64_t key, uint64_t index) {
    uint64_t b = tgo_splitmix64(key + index * 0xD1B54A32D192ED03ull);
    float u1 = (float)((b >> 40) + 1u) * 5.96046448e-08f;          /* 2^-24 */
    float u2 = (float)((b >> 16) & 0xFFFFFFu) * 5.96046448e-08f;
    float rad = sqrtf(-2.0f * tgo_ln_unit(u1));
    return rad * tgo_cos2pi(u2);
}

void tgo_synth_normal(uint64_t seed, uint64_t stream, float sigma, size_t n,
                      float *out) {
    uint64_t key = tgo_stream_key(seed, stream);
    #pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; i++)
        out[i] = sigma * tgo_normal_at(key, (uint64_t)i);
}

/* rows x cols weights N(0, sigma) quantized to Q4_0 (element (r, c) is draw
 * r*cols + c of the stream). */
void tgo_synth_q40(uint64_t seed, uint64_t stream, float sigma, int rows,
                   int cols, uint8_t *out) {
    uint64_t key = tgo_stream_key(seed, stream);
    int nb = cols / TGO_QK;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        float v[TGO_QK];
        for (int b = 0; b < nb; b++) {
            uint64_t base = (uint64_t)r * (uint64_t)cols + (uint64_t)b * TGO_QK;
            for (int j = 0; j < TGO_QK; j++)
                v[j] = sigma * tgo_normal_at(key, base + (uint64_t)j);
            tgo_quantize_q4_0(v, TGO_QK, out + ((size_t)r * nb + b) * TGO_Q40_BYTES);
        }
    }
}

/* ------------------------------------------------------------------ */
/* Q4_0 / Q8_0                                                          */
/* ------------------------------------------------------------------ */

/* Q4_0 quantizer (D1): the signed value m of largest magnitude (first one on
 * ties), d = m / -8, q = min(15, trunc(x / d + 8.5)), d stored as half.
 * The reference never quantizes weights (relayout.py:136 copies GGUF bytes);
 * this is the ggml block_q4_0 rule.  Pinned by
 * tests/test_oracle_formats.py::test_q4_0_* (independent numpy quantizer,
 * all-zero block, clamp at +max, dequantization error bound). */
void tgo_quantize_q4_0(const float *x, size_t n, uint8_t *out) {
    size_t nb = n / TGO_QK;
    for (size_t b = 0; b < nb; b++) {
        const float *xb = x + b * TGO_QK;
        uint8_t *o = out + b * TGO_Q40_BYTES;
        float amax = 0.0f, vmax = 0.0f;
        for (int j = 0; j < TGO_QK; j++) {
            float a = fabsf(xb[j]);
            if (amax < a) { amax = a; vmax = xb[j]; }
        }
        float d = vmax / -8.0f;
        float id = (d != 0.0f) ? 1.0f / d : 0.0f;
        wr16(o, tgo_f32_to_f16(d));
        for (int j = 0; j < 16; j++) {
            int q0 = (int)(xb[j] * id + 8.5f);
            int q1 = (int)(xb[j + 16] * id + 8.5f);
            if (q0 > 15) q0 = 15;
            if (q1 > 15) q1 = 15;
            o[2 + j] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

void tgo_dequantize_q4_0(const uint8_t *q, size_t n, float *out) {
    size_t nb = n / TGO_QK;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = q + b * TGO_Q40_BYTES;
        float d = tgo_f16_to_f32(rd16(blk));
        for (int j = 0; j < 16; j++) {
            out[b * TGO_QK + j] = d * (float)((blk[2 + j] & 15) - 8);
            out[b * TGO_QK + j + 16] = d * (float)((blk[2 + j] >> 4) - 8);
        }
    }
}

/* Q8_0 quantizer (D2), the arithmetic of libtinygiant.c:61-89 on blocks of
 * 32 with a half scale: amax = max|x|, d = amax/127, inv = 127/amax (0 when
 * amax = 0), q = round-half-even(x * inv) (vcvtnq_s32_f32, :81).  Pinned by
 * tests/test_oracle_formats.py::test_q8_0_* (numpy restatement, amax = 0,
 * +-amax -> +-127, exact half-way cases). */
void tgo_quantize_q8_0(const float *x, size_t n, uint8_t *out) {
    size_t nb = n / TGO_QK;
    for (size_t b = 0; b < nb; b++) {
        const float *xb = x + b * TGO_QK;
        uint8_t *o = out + b * TGO_Q80_BYTES;
        float amax = 0.0f;
        for (int j = 0; j < TGO_QK; j++) {
            float a = fabsf(xb[j]);
            amax = a > amax ? a : amax;
        }
        float d = amax / 127.0f;
        float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
        wr16(o, tgo_f32_to_f16(d));
        for (int j = 0; j < TGO_QK; j++)
            o[2 + j] = (uint8_t)(int8_t)(int)rintf(xb[j] * inv);
    }
}

void tgo_dequantize_q8_0(const uint8_t *q, size_t n, float *out) {
    size_t nb = n / TGO_QK;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = q + b * TGO_Q80_BYTES;
        float d = tgo_f16_to_f32(rd16(blk));
        for (int j = 0; j < TGO_QK; j++)
            out[b * TGO_QK + j] = d * (float)(int8_t)blk[2 + j];
    }
}

/* Exact int32 block sum S = sum_i (q_w,i - 8) * q_x,i, |S| <= 32,512 (D3);
 * the role of the vdotq_s32 groups in libtinygiant.c:135-158.  Pinned by
 * tests/test_oracle_formats.py::test_block_dot_bruteforce (numpy int64) and
 * the identity sum (q-8)x = sum qx - 8 sum x. */
int32_t tgo_block_dot_q40_q80(const uint8_t *w, const uint8_t *x) {
    int32_t s = 0;
    for (int j = 0; j < 16; j++) {
        int lo = (w[2 + j] & 15) - 8;
        int hi = (w[2 + j] >> 4) - 8;
        s += lo * (int8_t)x[2 + j] + hi * (int8_t)x[2 + 16 + j];
    }
    return s;
}

void tgo_block_sums(const uint8_t *W, int rows, int cols, const uint8_t *xq,
                    int32_t *sums) {
    int nb = cols / TGO_QK;
    for (int r = 0; r < rows; r++)
        for (int b = 0; b < nb; b++)
            sums[(size_t)r * nb + b] = tgo_block_dot_q40_q80(
                W + ((size_t)r * nb + b) * TGO_Q40_BYTES, xq + (size_t)b * TGO_Q80_BYTES);
}

/* Row dot (D3): acc = fma(round(S_b * dw_b), dx_b, acc) for b = 0..nb-1,
 * acc starting at 0.  Follows the per-block accumulation of
 * libtinygiant.c:109-167 (int dot, then fp32 scale into a running total).
 * Pinned by tests/test_oracle_formats.py::test_row_dot_* (float64 dequantized
 * dot within the rounding bound; explicit per-block loop in Python). */
float tgo_row_dot_q40_q80(const uint8_t *wrow, const uint8_t *xq, int nb) {
    float acc = 0.0f;
    for (int b = 0; b < nb; b++) {
        const uint8_t *w = wrow + (size_t)b * TGO_Q40_BYTES;
        const uint8_t *x = xq + (size_t)b * TGO_Q80_BYTES;
        int32_t s = tgo_block_dot_q40_q80(w, x);
        float u = (float)s * tgo_f16_to_f32(rd16(w));
        acc = fmaf(u, tgo_f16_to_f32(rd16(x)), acc);
    }
    return acc;
}

/* Q4_0 matrix x Q8_0 vector (role of matmul_q4k, libtinygiant.c:173-185). */
void tgo_matvec_q40(const uint8_t *W, int rows, int cols, const uint8_t *xq,
                    float *out) {
    int nb = cols / TGO_QK;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++)
        out[r] = tgo_row_dot_q40_q80(W + (size_t)r * nb * TGO_Q40_BYTES, xq, nb);
}

/* Tensor-planar arrangement of a [rows x nb] Q4_0 tensor in the same bytes:
 * all 16-byte nibble groups in (row, block) order, then all half scales.
 * Pinned by tests/test_oracle_formats.py::test_planar_roundtrip. */
void tgo_q40_to_planar(const uint8_t *aos, int rows, int nb, uint8_t *pl) {
    size_t n = (size_t)rows * nb;
    for (size_t i = 0; i < n; i++) {
        memcpy(pl + i * 16, aos + i * TGO_Q40_BYTES + 2, 16);
        memcpy(pl + n * 16 + i * 2, aos + i * TGO_Q40_BYTES, 2);
    }
}

void tgo_q40_from_planar(const uint8_t *pl, int rows, int nb, uint8_t *aos) {
    size_t n = (size_t)rows * nb;
    for (size_t i = 0; i < n; i++) {
        memcpy(aos + i * TGO_Q40_BYTES + 2, pl + i * 16, 16);
        memcpy(aos + i * TGO_Q40_BYTES, pl + n * 16 + i * 2, 2);
    }
}

/* ------------------------------------------------------------------ */
/* norm, router, SwiGLU                                                 */
/* ------------------------------------------------------------------ */


/* Sum of squares of x[0..n): fma chains over groups of 32 consecutive
 * elements (the rows one GPU block owns), then the group sums added in
 * ascending group order.  Role of the vfmaq loop in tg_rms_norm,
 * libtinygiant.c:324-331.  Pinned by tests/test_oracle_math.py::
 * test_sumsq_grouped (float64 bound; numpy restatement of the grouping). */
float tgo_sumsq(const float *x, int n) {
    float tot = 0.0f;
    for (int g = 0; g < n / 32; g++) {
        float a = 0.0f;
        for (int i = 0; i < 32; i++) a = fmaf(x[32 * g + i], x[32 * g + i], a);
        tot = tot + a;
    }
    return tot;
}

/* 1 / sqrt(mean(x^2) + eps) (libtinygiant.c:332; unit norm weight, D7). */
float tgo_rms_scale(const float *x, int n, float eps) {
    float ss = tgo_sumsq(x, n);
    return 1.0f / sqrtf(ss / (float)n + eps);
}

/* Un-normalised router dot w . x in the grouped order of tgo_sumsq: fma
 * chain inside each group of 32, groups added in ascending order.  The
 * logit is this value times the norm scale s: routers @ (x * s)
 * (engine.py:229-231) evaluated as s * (routers @ x), which lets the GPU
 * form the per-group partial sums where x is produced.  Pinned by
 * tests/test_oracle_math.py::test_router_dot_grouped. */
float tgo_router_dot(const float *w, const float *x, int n) {
    float tot = 0.0f;
    for (int g = 0; g < n / 32; g++) {
        float a = 0.0f;
        for (int i = 0; i < 32; i++) a = fmaf(w[32 * g + i], x[32 * g + i], a);
        tot = tot + a;
    }
    return tot;
}

void tgo_router_logits(const float *Wr, int E, int H, const float *x, float s,
                       float *logits) {
    for (int e = 0; e < E; e++) logits[e] = tgo_router_dot(Wr + (size_t)e * H, x, H) * s;
}

/* Router over rms_norm(x) * g (engine.py:229-231 with ffn_norms[i]):
 * routers @ ((x * s) * g) evaluated as s * ((w * g) . x), the norm weight
 * folded into each router column with one rounding (w[i] * g[i]) and the
 * dot in the grouped order of tgo_router_dot.  g = NULL is the unit
 * weight.  Pinned by tests/test_oracle_math.py::test_norm_weight_*. */
float tgo_router_dot_g(const float *w, const float *g, const float *x, int n) {
    if (!g) return tgo_router_dot(w, x, n);
    float tot = 0.0f;
    for (int gi = 0; gi < n / 32; gi++) {
        float a = 0.0f;
        for (int i = 0; i < 32; i++) {
            const int j = 32 * gi + i;
            const float wg = w[j] * g[j];
            a = fmaf(wg, x[j], a);
        }
        tot = tot + a;
    }
    return tot;
}

/* numpy's pairwise float32 sum (np.sum as used at engine.py:236) for the
 * short arrays that occur here (n <= 128). */
static float np_pairwise_sum(const float *a, int n) {
    if (n < 8) {
        float r = 0.0f;
        for (int i = 0; i < n; i++) r = r + a[i];
        return r;
    }
    float r[8];
    for (int j = 0; j < 8; j++) r[j] = a[j];
    int i;
    for (i = 8; i < n - (n % 8); i += 8)
        for (int j = 0; j < 8; j++) r[j] = r[j] + a[i + j];
    float res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (; i < n; i++) res = res + a[i];
    return res;
}

/* Top-k with renormalised softmax (engine.py:231-236).  idx/w are returned
 * in descending logit order; equal logits rank the lower expert index first
 * (np.argsort is unstable there, so this tie rule is this build's
 * definition).  The softmax runs over the k values in ascending order, as
 * np.argsort(...)[-k:] presents them.  Pinned by
 * tests/test_oracle_math.py::test_topk_* (brute-force sort, constructed
 * ties, weights sum to 1, equal to the renormalised full softmax). */
void tgo_topk_softmax(const float *logits, int E, int k, int32_t *idx,
                      float *w) {
    unsigned char taken[4096];
    memset(taken, 0, (size_t)E);
    for (int r = 0; r < k; r++) {
        int best = -1;
        for (int e = 0; e < E; e++) {
            if (taken[e]) continue;
            /* a NaN logit ranks below every number (as -inf) */
            float ve = logits[e] != logits[e] ? -INFINITY : logits[e];
            float vb = best < 0 ? 0.0f : (logits[best] != logits[best] ? -INFINITY : logits[best]);
            if (best < 0 || ve > vb) best = e;
        }
        taken[best] = 1;
        idx[r] = best;
    }
    float lmax = logits[idx[0]];
    float ex[64];
    for (int i = 0; i < k; i++) ex[i] = tgo_expf(logits[idx[k - 1 - i]] - lmax);
    float sum = np_pairwise_sum(ex, k);
    for (int i = 0; i < k; i++) w[k - 1 - i] = ex[i] / sum;
}

/* SiLU(g) * u (libtinygiant.c:580-583). */
float tgo_silu_mul(float g, float u) {
    float e = tgo_expf(-g);
    float s = g / (1.0f + e);
    return s * u;
}

/* ------------------------------------------------------------------ */
/* expert, layer, stack                                                 */
/* ------------------------------------------------------------------ */

/* One Q4_0 expert on a Q8_0 activation (role of tg_expert_forward,
 * libtinygiant.c:555-595): gate and up rows, SiLU*up, Q8_0 of h, down rows.
 * Any output pointer may be NULL. */
void tgo_expert_q40(const uint8_t *expert, int H, int I, const uint8_t *xq,
                    float *gate, float *up, float *h, uint8_t *hq,
                    float *down) {
    int nbh = H / TGO_QK, nbi = I / TGO_QK;
    size_t gate_bytes = (size_t)I * nbh * TGO_Q40_BYTES;
    const uint8_t *wg = expert, *wu = expert + gate_bytes, *wd = expert + 2 * gate_bytes;
    float *g = (float *)malloc(sizeof(float) * (size_t)I);
    float *u = (float *)malloc(sizeof(float) * (size_t)I);
    float *hh = (float *)malloc(sizeof(float) * (size_t)I);
    uint8_t *hqq = (uint8_t *)malloc((size_t)nbi * TGO_Q80_BYTES);
    for (int r = 0; r < I; r++) {
        g[r] = tgo_row_dot_q40_q80(wg + (size_t)r * nbh * TGO_Q40_BYTES, xq, nbh);
        u[r] = tgo_row_dot_q40_q80(wu + (size_t)r * nbh * TGO_Q40_BYTES, xq, nbh);
        hh[r] = tgo_silu_mul(g[r], u[r]);
    }
    tgo_quantize_q8_0(hh, (size_t)I, hqq);
    if (down)
        for (int r = 0; r < H; r++)
            down[r] = tgo_row_dot_q40_q80(wd + (size_t)r * nbi * TGO_Q40_BYTES, hqq, nbi);
    if (gate) memcpy(gate, g, sizeof(float) * (size_t)I);
    if (up) memcpy(up, u, sizeof(float) * (size_t)I);
    if (h) memcpy(h, hh, sizeof(float) * (size_t)I);
    if (hq) memcpy(hq, hqq, (size_t)nbi * TGO_Q80_BYTES);
    free(g); free(u); free(hh); free(hqq);
}

/* One MoE block for n_tokens independent tokens (engine.py:229-258 with
 * Q4_0 experts): xn = (x * s) * g with s = 1 / rms(x) (eps) and g the FFN
 * norm weight (tg_rms_norm's order, libtinygiant.c:332-339; g = NULL is
 * the unit weight), logits = Wr xn (tgo_router_dot_g), top-k + softmax,
 * Q8_0(xn), the k experts, moe_out = sum_j w_j down_j in ascending logit
 * order.  Work is split over rows so the result does not depend on the
 * thread count.  idx/w/xq_out may be NULL. */
void tgo_moe_layer_q40(const uint8_t *layer, const float *Wr, const float *g,
                       int H, int I, int E, int k, float eps, const float *x,
                       int n_tokens, float *moe_out, int32_t *idx_out,
                       float *w_out, uint8_t *xq_out) {
    int nbh = H / TGO_QK, nbi = I / TGO_QK;
    size_t gate_bytes = (size_t)I * nbh * TGO_Q40_BYTES;
    size_t down_bytes = (size_t)H * nbi * TGO_Q40_BYTES;
    size_t expert_bytes = 2 * gate_bytes + down_bytes;
    float *xn = (float *)malloc(sizeof(float) * (size_t)H);
    float *logits = (float *)malloc(sizeof(float) * (size_t)E);
    uint8_t *xq = (uint8_t *)malloc((size_t)nbh * TGO_Q80_BYTES);
    float *gu = (float *)malloc(sizeof(float) * 2 * (size_t)k * I);
    float *hh = (float *)malloc(sizeof(float) * (size_t)k * I);
    uint8_t *hq = (uint8_t *)malloc((size_t)k * nbi * TGO_Q80_BYTES);
    int32_t idx[64];
    float w[64];
    for (int t = 0; t < n_tokens; t++) {
        const float *xt = x + (size_t)t * H;
        float s = tgo_rms_scale(xt, H, eps);
        for (int i = 0; i < H; i++) {
            const float v = xt[i] * s;
            xn[i] = g ? v * g[i] : v;
        }
        for (int e = 0; e < E; e++) logits[e] = tgo_router_dot_g(Wr + (size_t)e * H, g, xt, H) * s;
        tgo_topk_softmax(logits, E, k, idx, w);
        tgo_quantize_q8_0(xn, (size_t)H, xq);
        if (idx_out) memcpy(idx_out + (size_t)t * k, idx, sizeof(int32_t) * (size_t)k);
        if (w_out) memcpy(w_out + (size_t)t * k, w, sizeof(float) * (size_t)k);
        if (xq_out) memcpy(xq_out + (size_t)t * nbh * TGO_Q80_BYTES, xq, (size_t)nbh * TGO_Q80_BYTES);
        /* gate/up rows of all k experts */
        #pragma omp parallel for schedule(static)
        for (int jr = 0; jr < 2 * k * I; jr++) {
            int j = jr / (2 * I), rr = jr % (2 * I);
            const uint8_t *ex = layer + (size_t)idx[j] * expert_bytes;
            const uint8_t *row = ex + (size_t)rr * nbh * TGO_Q40_BYTES; /* up follows gate */
            gu[jr] = tgo_row_dot_q40_q80(row, xq, nbh);
        }
        for (int j = 0; j < k; j++) {
            for (int r = 0; r < I; r++)
                hh[(size_t)j * I + r] = tgo_silu_mul(gu[(size_t)j * 2 * I + r],
                                                     gu[(size_t)j * 2 * I + I + r]);
            tgo_quantize_q8_0(hh + (size_t)j * I, (size_t)I, hq + (size_t)j * nbi * TGO_Q80_BYTES);
        }
        /* down rows and the weighted combine */
        float *out = moe_out + (size_t)t * H;
        #pragma omp parallel for schedule(static)
        for (int r = 0; r < H; r++) {
            float acc = 0.0f;
            for (int jj = k - 1; jj >= 0; jj--) {
                const uint8_t *wd = layer + (size_t)idx[jj] * expert_bytes + 2 * gate_bytes;
                float dv = tgo_row_dot_q40_q80(wd + (size_t)r * nbi * TGO_Q40_BYTES,
                                               hq + (size_t)jj * nbi * TGO_Q80_BYTES, nbi);
                acc = fmaf(w[jj], dv, acc);
            }
            out[r] = acc;
        }
    }
    free(xn); free(logits); free(xq); free(gu); free(hh); free(hq);
}

/* Layer stack (D7): x <- x + MoE_l(x) for l = 0..n_layers-1, each token
 * independent (engine.py:199-258 without attention).  norms (may be NULL,
 * as may each entry) holds each layer's FFN norm weight.  idx_trace (may be
 * NULL) receives [n_layers][n_tokens][k] expert ids. */
void tgo_moe_stack_q40(const uint8_t *const *layers, const float *const *routers,
                       const float *const *norms, int n_layers, int H, int I,
                       int E, int k, float eps, float *x, int n_tokens,
                       int32_t *idx_trace) {
    float *mo = (float *)malloc(sizeof(float) * (size_t)H * n_tokens);
    for (int l = 0; l < n_layers; l++) {
        tgo_moe_layer_q40(layers[l], routers[l], norms ? norms[l] : NULL, H, I, E, k, eps, x, n_tokens, mo,
                          idx_trace ? idx_trace + (size_t)l * n_tokens * k : NULL,
                          NULL, NULL);
        for (size_t i = 0; i < (size_t)H * n_tokens; i++) x[i] = x[i] + mo[i];
    }
    free(mo);
}

/* Token -> expert grouping for batched decode / prefill: counts[e], exclusive
 * offsets[e] (E+1 entries), and perm listing the (token*k + slot) pairs of
 * expert 0, then expert 1, ..., each list in ascending (token, slot) order.
 * Returns the number of experts with a non-empty group.  Pinned by
 * tests/test_oracle_math.py::test_group_by_expert (numpy stable argsort). */
int tgo_group_by_expert(const int32_t *idx, int n_tokens, int k, int E,
                        int32_t *counts, int32_t *offsets, int32_t *perm) {
    int n = n_tokens * k;
    for (int e = 0; e < E; e++) counts[e] = 0;
    for (int i = 0; i < n; i++) counts[idx[i]]++;
    offsets[0] = 0;
    int uniq = 0;
    for (int e = 0; e < E; e++) {
        offsets[e + 1] = offsets[e] + counts[e];
        uniq += counts[e] > 0;
    }
    int32_t *fill = (int32_t *)malloc(sizeof(int32_t) * (size_t)E);
    for (int e = 0; e < E; e++) fill[e] = offsets[e];
    for (int i = 0; i < n; i++) perm[fill[idx[i]]++] = i;
    free(fill);
    return uniq;
}

/* ------------------------------------------------------------------ */
/* legacy Q4_K / Q6_K / f16 functions                                   */
/* ------------------------------------------------------------------ */
/* These restate csrc/libtinygiant.c for the legacy ABI with contraction off
 * (the reference's FMA contraction under its own compiler is not
 * recoverable) and with tgo_expf in SiLU. */

/* quantize_q8, libtinygiant.c:61-89 (per-256 fp32 scale, RNE, int32 sum).
 * Pinned by tests/test_oracle_legacy.py::test_quantize_q8k. */
void tgo_quantize_q8k(const float *x, tgo_q8k_block *out, int n_blocks) {
    for (int b = 0; b < n_blocks; b++) {
        const float *xb = x + (size_t)b * 256;
        float amax = 0.0f;
        for (int i = 0; i < 256; i++) {
            float a = fabsf(xb[i]);
            amax = a > amax ? a : amax;
        }
        float inv = amax > 0 ? 127.0f / amax : 0.0f;
        out[b].scale = amax / 127.0f;
        int32_t sum = 0;
        for (int i = 0; i < 256; i++) {
            int32_t q = (int32_t)rintf(xb[i] * inv);
            out[b].qs[i] = (int8_t)(int16_t)q;
            sum += q;
        }
        out[b].sum = sum;
    }
}

/* get_scale_min_k4, libtinygiant.c:42-51 (6-bit scale/min pairs).  Pinned by
 * tests/test_oracle_legacy.py::test_scale_min_k4 (bit-field restatement). */
void tgo_scale_min_k4(int j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* dot_q4k_q8, libtinygiant.c:104-169.  Pinned by
 * tests/test_oracle_legacy.py::test_dot_q4k_* (reference tests 1a/2/3:
 * scalar Q8 reference, dequantize-then-dot). */
float tgo_dot_q4k_q8(const uint8_t *q4, const tgo_q8k_block *xq, int bpr) {
    float total = 0.0f;
    for (int b = 0; b < bpr; b++) {
        const uint8_t *bl = q4 + (size_t)b * 144;
        float d = tgo_f16_to_f32(rd16(bl)), dmin = tgo_f16_to_f32(rd16(bl + 2));
        const uint8_t *scales = bl + 4, *qs = bl + 16;
        const int8_t *x = xq[b].qs;
        float block_sum = 0.0f;
        for (int g = 0; g < 4; g++) {
            uint8_t sl, ml, sh, mh;
            tgo_scale_min_k4(2 * g, scales, &sl, &ml);
            tgo_scale_min_k4(2 * g + 1, scales, &sh, &mh);
            int32_t dl = 0, dh = 0, su_l = 0, su_h = 0;
            for (int j = 0; j < 32; j++) {
                uint8_t v = qs[g * 32 + j];
                dl += (v & 15) * x[g * 64 + j];
                dh += (v >> 4) * x[g * 64 + 32 + j];
                su_l += x[g * 64 + j];
                su_h += x[g * 64 + 32 + j];
            }
            float tl = (d * (float)sl) * (float)dl;
            float ul = (dmin * (float)ml) * (float)su_l;
            block_sum = block_sum + (tl - ul);
            float th = (d * (float)sh) * (float)dh;
            float uh = (dmin * (float)mh) * (float)su_h;
            block_sum = block_sum + (th - uh);
        }
        total = total + xq[b].scale * block_sum;
    }
    return total;
}

void tgo_matmul_q4k(const uint8_t *W, const float *x, float *y, int nrows, int ncols) {
    int bpr = ncols / 256;
    tgo_q8k_block *xq = (tgo_q8k_block *)malloc(sizeof(tgo_q8k_block) * (size_t)(bpr > 0 ? bpr : 1));
    tgo_quantize_q8k(x, xq, bpr);
    for (int r = 0; r < nrows; r++) y[r] = tgo_dot_q4k_q8(W + (size_t)r * bpr * 144, xq, bpr);
    free(xq);
}

/* dot_q6k_q8, libtinygiant.c:196-258.  Pinned by
 * tests/test_oracle_legacy.py::test_dot_q6k (dequantize-then-dot). */
float tgo_dot_q6k_q8(const uint8_t *q6, const tgo_q8k_block *xq, int bpr) {
    float total = 0.0f;
    for (int b = 0; b < bpr; b++) {
        const uint8_t *bl = q6 + (size_t)b * 210;
        const uint8_t *ql = bl, *qh = bl + 128;
        const int8_t *sc = (const int8_t *)(bl + 192);
        float d = tgo_f16_to_f32(rd16(bl + 208));
        const int8_t *x = xq[b].qs;
        float block_sum = 0.0f;
        for (int half = 0; half < 2; half++) {
            const uint8_t *qlh = ql + half * 64, *qhh = qh + half * 32;
            const int8_t *sch = sc + half * 8;
            const int8_t *xh = x + half * 128;
            for (int l = 0; l < 32; l += 16) {
                int is = l / 16;
                int32_t d1 = 0, d2 = 0, d3 = 0, d4 = 0;
                for (int kk = 0; kk < 16; kk++) {
                    int j = l + kk;
                    int hb = qhh[j];
                    int v1 = ((qlh[j] & 0xF) | (((hb >> 0) & 3) << 4)) - 32;
                    int v2 = ((qlh[j + 32] & 0xF) | (((hb >> 2) & 3) << 4)) - 32;
                    int v3 = ((qlh[j] >> 4) | (((hb >> 4) & 3) << 4)) - 32;
                    int v4 = ((qlh[j + 32] >> 4) | (((hb >> 6) & 3) << 4)) - 32;
                    d1 += v1 * xh[j];
                    d2 += v2 * xh[j + 32];
                    d3 += v3 * xh[j + 64];
                    d4 += v4 * xh[j + 96];
                }
                block_sum = block_sum + (float)sch[is + 0] * (float)d1;
                block_sum = block_sum + (float)sch[is + 2] * (float)d2;
                block_sum = block_sum + (float)sch[is + 4] * (float)d3;
                block_sum = block_sum + (float)sch[is + 6] * (float)d4;
            }
        }
        total = total + (d * xq[b].scale) * block_sum;
    }
    return total;
}

void tgo_matmul_q6k(const uint8_t *W, const float *x, float *y, int nrows, int ncols) {
    int bpr = ncols / 256;
    tgo_q8k_block *xq = (tgo_q8k_block *)malloc(sizeof(tgo_q8k_block) * (size_t)(bpr > 0 ? bpr : 1));
    tgo_quantize_q8k(x, xq, bpr);
    for (int r = 0; r < nrows; r++) y[r] = tgo_dot_q6k_q8(W + (size_t)r * bpr * 210, xq, bpr);
    free(xq);
}

/* Two 4-lane fma accumulators over 8-element steps, lanes added, pairwise
 * horizontal sum, scalar tail (libtinygiant.c:277-318). */
static float dot_two_acc(const uint16_t *ah, const float *af, const float *x, int n) {
    float a0[4] = {0, 0, 0, 0}, a1[4] = {0, 0, 0, 0};
    int i = 0;
    for (; i + 7 < n; i += 8)
        for (int c = 0; c < 4; c++) {
            float w0 = ah ? tgo_f16_to_f32(ah[i + c]) : af[i + c];
            float w1 = ah ? tgo_f16_to_f32(ah[i + 4 + c]) : af[i + 4 + c];
            a0[c] = fmaf(w0, x[i + c], a0[c]);
            a1[c] = fmaf(w1, x[i + 4 + c], a1[c]);
        }
    float t[4];
    for (int c = 0; c < 4; c++) t[c] = a0[c] + a1[c];
    float sum = (t[0] + t[1]) + (t[2] + t[3]);
    for (; i < n; i++) sum = sum + (ah ? tgo_f16_to_f32(ah[i]) : af[i]) * x[i];
    return sum;
}

/* matvec_f16, libtinygiant.c:277-295.  Pinned by
 * tests/test_oracle_legacy.py::test_matvec_f16_f32 (float64 bound). */
void tgo_matvec_f16(const uint16_t *A, const float *x, float *y, int nrows, int ncols) {
    for (int r = 0; r < nrows; r++) y[r] = dot_two_acc(A + (size_t)r * ncols, NULL, x, ncols);
}

/* tg_f32_matvec, libtinygiant.c:304-318. */
void tgo_matvec_f32(const float *A, const float *x, float *y, int nrows, int ncols) {
    for (int r = 0; r < nrows; r++) y[r] = dot_two_acc(NULL, A + (size_t)r * ncols, x, ncols);
}

/* tg_rms_norm, libtinygiant.c:322-340.  Pinned by
 * tests/test_oracle_legacy.py::test_rms_norm (float64 bound). */
void tgo_rms_norm(const float *x, const float *w, float *out, int dim, float eps) {
    float v[4] = {0, 0, 0, 0};
    int i = 0;
    for (; i + 3 < dim; i += 4)
        for (int c = 0; c < 4; c++) v[c] = fmaf(x[i + c], x[i + c], v[c]);
    float ss = (v[0] + v[1]) + (v[2] + v[3]);
    for (; i < dim; i++) ss = ss + x[i] * x[i];
    float scale = 1.0f / sqrtf(ss / (float)dim + eps);
    for (i = 0; i < dim; i++) out[i] = (x[i] * scale) * w[i];
}

/* tg_expert_forward_mixed, libtinygiant.c:599-643 (down_format 0 = Q4_K,
 * 1 = f16, 2 = Q6_K); output accumulates weight * down. */
void tgo_expert_forward_mixed(const uint8_t *gate, const uint8_t *up,
                              const void *down, int down_format,
                              const float *in, float *out, float weight,
                              int embed, int inter) {
    int gbpr = embed / 256, dbpr = inter / 256;
    tgo_q8k_block *xq = (tgo_q8k_block *)malloc(sizeof(tgo_q8k_block) * (size_t)(gbpr > 0 ? gbpr : 1));
    tgo_quantize_q8k(in, xq, gbpr);
    float *hid = (float *)malloc(sizeof(float) * (size_t)inter);
    float *dn = (float *)malloc(sizeof(float) * (size_t)embed);
    for (int r = 0; r < inter; r++) {
        float g = tgo_dot_q4k_q8(gate + (size_t)r * gbpr * 144, xq, gbpr);
        float u = tgo_dot_q4k_q8(up + (size_t)r * gbpr * 144, xq, gbpr);
        hid[r] = tgo_silu_mul(g, u);
    }
    if (down_format == 1) {
        tgo_matvec_f16((const uint16_t *)down, hid, dn, embed, inter);
    } else if (down_format == 2) {
        tgo_matmul_q6k((const uint8_t *)down, hid, dn, embed, inter);
    } else {
        tgo_q8k_block *hq = (tgo_q8k_block *)malloc(sizeof(tgo_q8k_block) * (size_t)(dbpr > 0 ? dbpr : 1));
        tgo_quantize_q8k(hid, hq, dbpr);
        for (int r = 0; r < embed; r++)
            dn[r] = tgo_dot_q4k_q8((const uint8_t *)down + (size_t)r * dbpr * 144, hq, dbpr);
        free(hq);
    }
    for (int i = 0; i < embed; i++) out[i] = out[i] + weight * dn[i];
    free(xq); free(hid); free(dn);
}

/* tg_moe_forward, libtinygiant.c:647-655 (all-Q4_K experts, gate|up|down
 * contiguous; output zeroed first). */
void tgo_moe_forward_q4k(const uint8_t *const *experts, const float *w, int n,
                         const float *in, float *out, int embed, int inter) {
    size_t gate_bytes = (size_t)inter * (embed / 256) * 144;
    for (int i = 0; i < embed; i++) out[i] = 0.0f;
    for (int e = 0; e < n; e++)
        tgo_expert_forward_mixed(experts[e], experts[e] + gate_bytes,
                                 experts[e] + 2 * gate_bytes, 0, in, out, w[e],
                                 embed, inter);
}

/* dot_q4k_scalar / tg_matmul_q4k_scalar, libtinygiant.c:706-741. */
void tgo_matmul_q4k_scalar(const uint8_t *W, const float *x, float *y, int nrows, int ncols) {
    int bpr = ncols / 256;
    for (int r = 0; r < nrows; r++) {
        float total = 0.0f;
        const uint8_t *q4 = W + (size_t)r * bpr * 144;
        for (int b = 0; b < bpr; b++) {
            const uint8_t *bl = q4 + (size_t)b * 144;
            float d = tgo_f16_to_f32(rd16(bl)), dmin = tgo_f16_to_f32(rd16(bl + 2));
            const uint8_t *qs = bl + 16;
            const float *xb = x + (size_t)b * 256;
            for (int g = 0; g < 4; g++) {
                uint8_t sl, ml, sh, mh;
                tgo_scale_min_k4(2 * g, bl + 4, &sl, &ml);
                tgo_scale_min_k4(2 * g + 1, bl + 4, &sh, &mh);
                for (int j = 0; j < 32; j++) {
                    uint8_t v = qs[g * 32 + j];
                    float vl = (d * (float)sl) * (float)(v & 0xF) - dmin * (float)ml;
                    float vh = (d * (float)sh) * (float)(v >> 4) - dmin * (float)mh;
                    total = total + (vl * xb[g * 64 + j] + vh * xb[g * 64 + 32 + j]);
                }
            }
        }
        y[r] = total;
    }
}

/* dequant_q4k_block, csrc/test_libtinygiant.c:80-99. */
void tgo_dequant_q4k_block(const uint8_t *block, float *out) {
    float d = tgo_f16_to_f32(rd16(block)), dmin = tgo_f16_to_f32(rd16(block + 2));
    const uint8_t *qs = block + 16;
    for (int g = 0; g < 4; g++) {
        uint8_t sl, ml, sh, mh;
        tgo_scale_min_k4(2 * g, block + 4, &sl, &ml);
        tgo_scale_min_k4(2 * g + 1, block + 4, &sh, &mh);
        for (int j = 0; j < 32; j++) {
            uint8_t v = qs[g * 32 + j];
            out[g * 64 + j] = (d * (float)sl) * (float)(v & 0xF) - dmin * (float)ml;
            out[g * 64 + 32 + j] = (d * (float)sh) * (float)(v >> 4) - dmin * (float)mh;
        }
    }
}

/* Q6_K dequantization implied by dot_q6k_q8's unpacking
 * (libtinygiant.c:211-253): element half*128 + 32*m + j has scale
 * sc[half*8 + j/16 + 2m]. */
void tgo_dequant_q6k_block(const uint8_t *block, float *out) {
    const uint8_t *ql = block, *qh = block + 128;
    const int8_t *sc = (const int8_t *)(block + 192);
    float d = tgo_f16_to_f32(rd16(block + 208));
    for (int half = 0; half < 2; half++)
        for (int j = 0; j < 32; j++) {
            int hb = qh[half * 32 + j];
            int lo0 = ql[half * 64 + j], lo1 = ql[half * 64 + j + 32];
            int v[4];
            v[0] = ((lo0 & 0xF) | (((hb >> 0) & 3) << 4)) - 32;
            v[1] = ((lo1 & 0xF) | (((hb >> 2) & 3) << 4)) - 32;
            v[2] = ((lo0 >> 4) | (((hb >> 4) & 3) << 4)) - 32;
            v[3] = ((lo1 >> 4) | (((hb >> 6) & 3) << 4)) - 32;
            for (int m = 0; m < 4; m++)
                out[half * 128 + 32 * m + j] = d * (float)sc[half * 8 + j / 16 + 2 * m] * (float)v[m];
        }
}

/* apply_rope_inplace, libtinygiant.c:344-361: per head, pairs (i, i + half)
 * rotated by the table row of `pos`: x1' = x1 c - x2 s (vmlsq_f32: product,
 * product, difference, each rounded) and x2' = fma(x1, s, x2 c) (vfmaq_f32 on
 * the rounded x2 c).  half is a multiple of 4 (the reference steps by 4). */
void tgo_rope(float *x, int n_heads, int head_dim, const float *cos_t, const float *sin_t, int pos) {
    int half = head_dim / 2;
    const float *c = cos_t + (size_t)pos * half, *sn = sin_t + (size_t)pos * half;
    for (int h = 0; h < n_heads; h++) {
        float *xh = x + (size_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            float x1 = xh[i], x2 = xh[half + i];
            float a = x1 * c[i], b = x2 * sn[i];
            xh[i] = a - b;
            xh[half + i] = fmaf(x1, sn[i], x2 * c[i]);
        }
    }
}

/* One head's scores, softmax and weighted values (libtinygiant.c:405-446):
 * dot = four fma lanes over steps of 4, (l0 + l1) + (l2 + l3) (vaddvq_f32),
 * the tail one product and add at a time; score = dot * inv_sqrt; e =
 * exp(score - max) added in order; out[d] = fma chain over t of
 * (e_t * inv_sum) v_t[d] (vfmaq_f32; the tail d unfused). */
static void attn_head(const float *q, const float *kc, const float *vc, int seq, int hd, float inv_sqrt,
                      float *out, float *scores) {
    float mx = -1e30f;
    for (int t = 0; t < seq; t++) {
        const float *kt = kc + (size_t)t * hd;
        float acc[4] = {0, 0, 0, 0};
        int d = 0;
        for (; d + 3 < hd; d += 4)
            for (int l = 0; l < 4; l++) acc[l] = fmaf(q[d + l], kt[d + l], acc[l]);
        float dot = (acc[0] + acc[1]) + (acc[2] + acc[3]);
        for (; d < hd; d++) dot = dot + q[d] * kt[d];
        scores[t] = dot * inv_sqrt;
        if (scores[t] > mx) mx = scores[t];
    }
    float sum = 0.0f;
    for (int t = 0; t < seq; t++) {
        scores[t] = tgo_expf(scores[t] - mx);
        sum = sum + scores[t];
    }
    float inv_sum = 1.0f / sum;
    for (int d = 0; d < hd; d++) out[d] = 0.0f;
    int hd4 = hd & ~3;
    for (int t = 0; t < seq; t++) {
        float w = scores[t] * inv_sum;
        const float *vt = vc + (size_t)t * hd;
        for (int d = 0; d < hd4; d++) out[d] = fmaf(w, vt[d], out[d]);
        for (int d = hd4; d < hd; d++) out[d] = out[d] + w * vt[d];
    }
}

/* tg_attention_decode (f32 weights, libtinygiant.c:365-457) and
 * tg_attention_decode_q4 (Q4_K q / k / o, f16 v, :460-551): projections,
 * per-head RMS norms of q and k (eps 1e-6), RoPE, the new k (after RoPE) and
 * v appended to the caches [n_kv_heads][kv_max][head_dim] at kv_len, GQA
 * attention over kv_len + 1 positions, output projection. */
static void attn_decode(int q4, const void *wq, const void *wk, const void *wv, const void *wo,
                        const float *q_norm_w, const float *k_norm_w, float *kv_k, float *kv_v, int kv_len,
                        int kv_max, const float *rope_cos, const float *rope_sin, const float *input,
                        float *output, int embed, int n_heads, int n_kv_heads, int hd, int pos) {
    int q_dim = n_heads * hd, kv_dim = n_kv_heads * hd, ratio = n_heads / n_kv_heads;
    float *q = (float *)malloc(sizeof(float) * (size_t)q_dim), *k = (float *)malloc(sizeof(float) * (size_t)kv_dim);
    float *v = (float *)malloc(sizeof(float) * (size_t)kv_dim);
    float *qn = (float *)malloc(sizeof(float) * (size_t)q_dim), *kn = (float *)malloc(sizeof(float) * (size_t)kv_dim);
    float *ao = (float *)malloc(sizeof(float) * (size_t)q_dim);
    float *sc = (float *)malloc(sizeof(float) * (size_t)(kv_len + 1));
    if (q4) {
        tgo_matmul_q4k((const uint8_t *)wq, input, q, q_dim, embed);
        tgo_matmul_q4k((const uint8_t *)wk, input, k, kv_dim, embed);
        tgo_matvec_f16((const uint16_t *)wv, input, v, kv_dim, embed);
    } else {
        tgo_matvec_f32((const float *)wq, input, q, q_dim, embed);
        tgo_matvec_f32((const float *)wk, input, k, kv_dim, embed);
        tgo_matvec_f32((const float *)wv, input, v, kv_dim, embed);
    }
    for (int h = 0; h < n_heads; h++) tgo_rms_norm(q + (size_t)h * hd, q_norm_w, qn + (size_t)h * hd, hd, 1e-6f);
    for (int h = 0; h < n_kv_heads; h++) tgo_rms_norm(k + (size_t)h * hd, k_norm_w, kn + (size_t)h * hd, hd, 1e-6f);
    tgo_rope(qn, n_heads, hd, rope_cos, rope_sin, pos);
    tgo_rope(kn, n_kv_heads, hd, rope_cos, rope_sin, pos);
    for (int h = 0; h < n_kv_heads; h++) {
        memcpy(kv_k + ((size_t)h * kv_max + kv_len) * hd, kn + (size_t)h * hd, sizeof(float) * (size_t)hd);
        memcpy(kv_v + ((size_t)h * kv_max + kv_len) * hd, v + (size_t)h * hd, sizeof(float) * (size_t)hd);
    }
    float inv_sqrt = 1.0f / sqrtf((float)hd);
    for (int h = 0; h < n_heads; h++) {
        int kh = h / ratio;
        attn_head(qn + (size_t)h * hd, kv_k + (size_t)kh * kv_max * hd, kv_v + (size_t)kh * kv_max * hd, kv_len + 1,
                  hd, inv_sqrt, ao + (size_t)h * hd, sc);
    }
    if (q4)
        tgo_matmul_q4k((const uint8_t *)wo, ao, output, embed, q_dim);
    else
        tgo_matvec_f32((const float *)wo, ao, output, embed, q_dim);
    free(q); free(k); free(v); free(qn); free(kn); free(ao); free(sc);
}

void tgo_attention_decode(const float *wq, const float *wk, const float *wv, const float *wo,
                          const float *q_norm_w, const float *k_norm_w, float *kv_k, float *kv_v, int kv_len,
                          int kv_max, const float *rope_cos, const float *rope_sin, const float *input,
                          float *output, int embed, int n_heads, int n_kv_heads, int head_dim, int pos) {
    attn_decode(0, wq, wk, wv, wo, q_norm_w, k_norm_w, kv_k, kv_v, kv_len, kv_max, rope_cos, rope_sin, input, output,
                embed, n_heads, n_kv_heads, head_dim, pos);
}

void tgo_attention_decode_q4(const uint8_t *wq, const uint8_t *wk, const uint16_t *wv, const uint8_t *wo,
                             const float *q_norm_w, const float *k_norm_w, float *kv_k, float *kv_v, int kv_len,
                             int kv_max, const float *rope_cos, const float *rope_sin, const float *input,
                             float *output, int embed, int n_heads, int n_kv_heads, int head_dim, int pos) {
    attn_decode(1, wq, wk, wv, wo, q_norm_w, k_norm_w, kv_k, kv_v, kv_len, kv_max, rope_cos, rope_sin, input, output,
                embed, n_heads, n_kv_heads, head_dim, pos);
}

/* tg_transformer_layer, libtinygiant.c:662-702: RMS norm (attn_norm_w),
 * f32 attention, x += attn; RMS norm (ffn_norm_w), the experts' forward
 * (down_is_f16[e] as the down format) accumulated from zero, x += moe. */
void tgo_transformer_layer(const float *wq, const float *wk, const float *wv, const float *wo,
                           const float *attn_norm_w, const float *q_norm_w, const float *k_norm_w,
                           const float *ffn_norm_w, float *kv_k, float *kv_v, int kv_len, int kv_max,
                           const float *rope_cos, const float *rope_sin, const uint8_t *const *gate_ptrs,
                           const uint8_t *const *up_ptrs, const void *const *down_ptrs, const int *down_is_f16,
                           const float *expert_weights, int n_active, float *x, int embed, int inter, int n_heads,
                           int n_kv_heads, int head_dim, int pos) {
    float *nrm = (float *)malloc(sizeof(float) * (size_t)embed), *ao = (float *)malloc(sizeof(float) * (size_t)embed);
    float *mo = (float *)malloc(sizeof(float) * (size_t)embed);
    tgo_rms_norm(x, attn_norm_w, nrm, embed, 1e-6f);
    tgo_attention_decode(wq, wk, wv, wo, q_norm_w, k_norm_w, kv_k, kv_v, kv_len, kv_max, rope_cos, rope_sin, nrm, ao,
                         embed, n_heads, n_kv_heads, head_dim, pos);
    for (int i = 0; i < embed; i++) x[i] = x[i] + ao[i];
    tgo_rms_norm(x, ffn_norm_w, nrm, embed, 1e-6f);
    for (int i = 0; i < embed; i++) mo[i] = 0.0f;
    for (int e = 0; e < n_active; e++)
        tgo_expert_forward_mixed(gate_ptrs[e], up_ptrs[e], down_ptrs[e], down_is_f16[e], nrm, mo, expert_weights[e],
                                 embed, inter);
    for (int i = 0; i < embed; i++) x[i] = x[i] + mo[i];
    free(nrm); free(ao); free(mo);
}

int tgo_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
#else
    (void)n;
    return 1;
#endif
}

int tgo_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
