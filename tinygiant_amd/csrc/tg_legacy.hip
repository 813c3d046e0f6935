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
__global__ __launch_bounds__(256) void k_quantize_q8k(const float *__restrict__ x, Q8K *__restrict__ out, int nblocks) {
    const int lane = threadIdx.x & 63, b = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nblocks) return;  // uniform over the wave
    const float4 v4 = reinterpret_cast<const float4 *>(x + (size_t)b * LG_QK)[lane];
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
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
    reinterpret_cast<uint32_t *>(out[b].qs)[lane] = packed;
    if (lane == 0) {
        out[b].scale = a / 127.0f;
        out[b].sum = s;
    }
}

// --------------------------------------------------------------- Q4_K dot
// y[r] = dot_q4k_q8(row r, xq), libtinygiant.c:104-169: per block, for each
// group g the integer dots of the 32 low and 32 high nibbles with their
// activations and the activations' sums, turned into
// (d sc_l) dl - (dmin m_l) su_l and (d sc_h) dh - (dmin m_h) su_h; the eight
// differences added in group order, blocks added in order as scale * sum.
// One wave per row; per pass four blocks, 16 lanes each (lane: group s / 4,
// bytes 8 (s % 4) .. +8 of its 32).
__global__ __launch_bounds__(256) void k_matmul_q4k(const uint8_t *__restrict__ W, const Q8K *__restrict__ xq,
                                                    float *__restrict__ y, int nrows, int bpr) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= nrows) return;  // uniform over the wave
    const int bq = lane >> 4, s = lane & 15, g = s >> 2, part = s & 3;
    const uint8_t *wr = W + (size_t)row * bpr * LG_Q4K_BYTES;
    float total = 0.0f;
    for (int b0 = 0; b0 < bpr; b0 += 4) {
        const int b = b0 + bq;
        const bool on = b < bpr;
        const uint8_t *bl = wr + (size_t)(on ? b : 0) * LG_Q4K_BYTES;
        int dl = 0, dh = 0, sul = 0, suh = 0;
        if (on) {
            const uint2 qv = *reinterpret_cast<const uint2 *>(bl + 16 + g * 32 + part * 8);
            const uint2 xl = *reinterpret_cast<const uint2 *>(xq[b].qs + g * 64 + part * 8);
            const uint2 xh = *reinterpret_cast<const uint2 *>(xq[b].qs + g * 64 + 32 + part * 8);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t v = ((i < 4 ? qv.x : qv.y) >> (8 * (i & 3))) & 0xFF;
                const int lo = byte_s8(i < 4 ? xl.x : xl.y, i & 3), hi = byte_s8(i < 4 ? xh.x : xh.y, i & 3);
                dl += (int)(v & 15) * lo;
                dh += (int)(v >> 4) * hi;
                sul += lo;
                suh += hi;
            }
        }
#pragma unroll
        for (int o = 1; o < 4; o <<= 1) {
            dl += __shfl_xor(dl, o, WAVE);
            dh += __shfl_xor(dh, o, WAVE);
            sul += __shfl_xor(sul, o, WAVE);
            suh += __shfl_xor(suh, o, WAVE);
        }
        float difl = 0.0f, difh = 0.0f;
        if (on) {
            const float d = h2f(ld16(bl)), dmin = h2f(ld16(bl + 2));
            int sl, ml, sh, mh;
            scale_min_k4(2 * g, bl + 4, sl, ml);
            scale_min_k4(2 * g + 1, bl + 4, sh, mh);
            const float tl = (d * (float)sl) * (float)dl, ul = (dmin * (float)ml) * (float)sul;
            const float th = (d * (float)sh) * (float)dh, uh = (dmin * (float)mh) * (float)suh;
            difl = tl - ul;
            difh = th - uh;
        }
        // block sum of block bq over its groups in order (lanes 16 bq + 4 g)
        float bs = 0.0f;
#pragma unroll
        for (int gg = 0; gg < 4; gg++) {
            const float a = __shfl(difl, bq * 16 + 4 * gg, WAVE), c = __shfl(difh, bq * 16 + 4 * gg, WAVE);
            bs = bs + a;
            bs = bs + c;
        }
        // the pass's blocks in order
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float bsq = __shfl(bs, 16 * q, WAVE);
            if (b0 + q < bpr) total = total + xq[b0 + q].scale * bsq;
        }
    }
    if (lane == 0) y[row] = total;
}

// --------------------------------------------------------------- Q6_K dot
// y[r] = dot_q6k_q8(row r, xq), libtinygiant.c:196-258: per block, for each
// half and each 16-element step `is` four integer dots d1..d4 of 6-bit
// values (low nibble | 2 high bits, minus 32) with activations 0, 32, 64 and
// 96 ahead; the sixteen products sc * d added in (half, is, 1..4) order;
// blocks added in order as (d * scale) * sum.  One wave per row; per pass
// four blocks, 16 lanes each (lane: half s / 8, step (s / 4) % 2, four of
// the step's 16 elements).
__global__ __launch_bounds__(256) void k_matmul_q6k(const uint8_t *__restrict__ W, const Q8K *__restrict__ xq,
                                                    float *__restrict__ y, int nrows, int bpr) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= nrows) return;  // uniform over the wave
    const int bq = lane >> 4, s = lane & 15, half = s >> 3, is = (s >> 2) & 1, part = s & 3;
    const uint8_t *wr = W + (size_t)row * bpr * LG_Q6K_BYTES;
    float total = 0.0f;
    for (int b0 = 0; b0 < bpr; b0 += 4) {
        const int b = b0 + bq;
        const bool on = b < bpr;
        const uint8_t *bl = wr + (size_t)(on ? b : 0) * LG_Q6K_BYTES;
        int d1 = 0, d2 = 0, d3 = 0, d4 = 0;
        if (on) {
            const uint8_t *ql = bl + half * 64, *qh = bl + 128 + half * 32;
            const int8_t *xh = xq[b].qs + half * 128;
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const int j = is * 16 + part * 4 + kk;
                const int hb = qh[j], l0 = ql[j], l1 = ql[j + 32];
                d1 += (((l0 & 0xF) | ((hb & 3) << 4)) - 32) * xh[j];
                d2 += (((l1 & 0xF) | (((hb >> 2) & 3) << 4)) - 32) * xh[j + 32];
                d3 += (((l0 >> 4) | (((hb >> 4) & 3) << 4)) - 32) * xh[j + 64];
                d4 += (((l1 >> 4) | (((hb >> 6) & 3) << 4)) - 32) * xh[j + 96];
            }
        }
#pragma unroll
        for (int o = 1; o < 4; o <<= 1) {
            d1 += __shfl_xor(d1, o, WAVE);
            d2 += __shfl_xor(d2, o, WAVE);
            d3 += __shfl_xor(d3, o, WAVE);
            d4 += __shfl_xor(d4, o, WAVE);
        }
        float t1 = 0.0f, t2 = 0.0f, t3 = 0.0f, t4 = 0.0f;
        if (on) {
            const int8_t *sc = reinterpret_cast<const int8_t *>(bl + 192) + half * 8;
            t1 = (float)sc[is] * (float)d1;
            t2 = (float)sc[is + 2] * (float)d2;
            t3 = (float)sc[is + 4] * (float)d3;
            t4 = (float)sc[is + 6] * (float)d4;
        }
        float bs = 0.0f;
#pragma unroll
        for (int st = 0; st < 4; st++) {  // (half, is) = (0,0), (0,1), (1,0), (1,1): lanes 16 bq + 4 st
            const int src = bq * 16 + 4 * st;
            bs = bs + __shfl(t1, src, WAVE);
            bs = bs + __shfl(t2, src, WAVE);
            bs = bs + __shfl(t3, src, WAVE);
            bs = bs + __shfl(t4, src, WAVE);
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float bsq = __shfl(bs, 16 * q, WAVE);
            if (b0 + q < bpr) {
                const float d = h2f(ld16(wr + (size_t)(b0 + q) * LG_Q6K_BYTES + 208));
                total = total + (d * xq[b0 + q].scale) * bsq;
            }
        }
    }
    if (lane == 0) y[row] = total;
}

// ------------------------------------------------------ f16 / f32 matvec
// matvec_f16 / tg_f32_matvec, libtinygiant.c:277-318: eight fma chains over
// steps of 8 elements (chain c takes elements i + c), t_c = chain c + chain
// c + 4, sum = (t0 + t1) + (t2 + t3), then the tail (ncols % 8) one product
// and one add at a time.  Eight lanes per row.
template <bool HALF>
__global__ __launch_bounds__(256) void k_matvec_two_acc(const void *__restrict__ A, const float *__restrict__ x,
                                                        float *__restrict__ y, int nrows, int ncols) {
    const int c = threadIdx.x & 7, row = (blockIdx.x * 256 + threadIdx.x) >> 3;
    const bool on = row < nrows;
    const int n8 = ncols & ~7;
    auto wat = [&](size_t i) -> float {
        return HALF ? h2f(reinterpret_cast<const uint16_t *>(A)[i]) : reinterpret_cast<const float *>(A)[i];
    };
    const size_t r0 = (size_t)(on ? row : 0) * ncols;
    float a = 0.0f;
    if (on) {
        int i = 0;
        for (; i + 32 <= n8; i += 32) {  // four steps' operands loaded ahead of the chain
            float w4[4], x4[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                w4[u] = wat(r0 + i + 8 * u + c);
                x4[u] = x[i + 8 * u + c];
            }
#pragma unroll
            for (int u = 0; u < 4; u++) a = __builtin_fmaf(w4[u], x4[u], a);
        }
        for (; i < n8; i += 8) a = __builtin_fmaf(wat(r0 + i + c), x[i + c], a);
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
// per row (row b at x + b * dim, the same weight w).
__global__ __launch_bounds__(256) void k_rms_norm(const float *__restrict__ x, const float *__restrict__ w,
                                                  float *__restrict__ out, int dim, float eps) {
    __shared__ float v[4];
    __shared__ float scale;
    const int tid = threadIdx.x, n4 = dim & ~3;
    x += (size_t)blockIdx.x * dim;
    out += (size_t)blockIdx.x * dim;
    if (tid < 4) {
        float a = 0.0f;
        for (int i = 0; i < n4; i += 4) a = __builtin_fmaf(x[i + tid], x[i + tid], a);
        v[tid] = a;
    }
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

// One head's attention over seq cached positions (libtinygiant.c:405-446):
// score_t = dot(q, k_t) * inv_sqrt, the dot in four fma lanes over steps of 4
// added as (l0 + l1) + (l2 + l3) with the tail one product and add at a time;
// e_t = exp(score_t - max); sum = e_0 + e_1 + ... in order; out[d] = fma
// chain over t of (e_t * (1 / sum)) v_t[d] (the tail d unfused).  One block
// per head (kv head h / ratio), 256 threads; scr: this head's seq scores
// (device scratch).  Rows of K and V pass through LDS in chunks of ATT_TC(hd)
// rows (K rows padded to hd + 1 floats, so the lanes reading different rows
// use different banks): per chunk two threads share a row's dot (lanes 0-1
// and 2-3), and in the weighted sum each thread carries its element's chain
// across the chunks.
__host__ __device__ inline int att_tc(int hd) {
    int tc = 16384 / (hd + 1);
    tc = tc > 128 ? 128 : tc;
    return tc & ~1;
}

__host__ __device__ inline size_t att_lds_bytes(int hd) { return 4 * ((size_t)att_tc(hd) * (hd + 1) + 1024); }

// n rows of hd floats (contiguous at src) into LDS rows of `stride` floats:
// every thread's loads of a round are in flight together (16 float4 when hd
// is a multiple of 4, else 16 floats), then stored.
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

__global__ __launch_bounds__(256) void k_attn_head(const float *__restrict__ q, const float *__restrict__ kc,
                                                   const float *__restrict__ vc, float *__restrict__ scr,
                                                   float *__restrict__ out, int seq, int hd, int ratio,
                                                   float inv_sqrt) {
    extern __shared__ __align__(16) float lds[];  // [TC][hd + 1] rows, then 1024 floats of weights
    __shared__ float qs[512];
    __shared__ float red[256];
    __shared__ float inv_sum;
    const int h = blockIdx.x, tid = threadIdx.x, kh = h / ratio, hd4 = hd & ~3, TC = att_tc(hd), ks = hd + 1;
    const float *qh = q + (size_t)h * hd;
    const float *kch = kc + (size_t)kh * seq * hd, *vch = vc + (size_t)kh * seq * hd;
    float *sc = scr + (size_t)h * seq;
    float *wl = lds + (size_t)TC * ks;
    for (int d = tid; d < hd; d += 256) qs[d] = qh[d];
    // 1. scores, a chunk of TC rows at a time: thread pair (row tid / 2, lanes 2 (tid % 2) .. +1)
    float mx = -1e30f;
    const int r = tid >> 1, hf = tid & 1;
    for (int t0 = 0; t0 < seq; t0 += TC) {
        const int n = min(TC, seq - t0);
        __syncthreads();  // the previous chunk's rows are read
        att_stage(lds, ks, kch + (size_t)t0 * hd, n, hd);
        __syncthreads();
        float a0 = 0.0f, a1 = 0.0f;
        if (r < n) {
            const float *kt = lds + r * ks;
#pragma unroll 8
            for (int d = 2 * hf; d < hd4; d += 4) {
                a0 = __builtin_fmaf(qs[d], kt[d], a0);
                a1 = __builtin_fmaf(qs[d + 1], kt[d + 1], a1);
            }
        }
        const float mine = a0 + a1, other = __shfl_xor(mine, 1, WAVE);
        if (r < n && hf == 0) {
            float dot = mine + other;  // (l0 + l1) + (l2 + l3)
            const float *kt = lds + r * ks;
            for (int d = hd4; d < hd; d++) dot = dot + qs[d] * kt[d];
            const float sv = dot * inv_sqrt;
            sc[t0 + r] = sv;
            mx = sv > mx ? sv : mx;
        }
    }
    red[tid] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) red[tid] = red[tid + o] > red[tid] ? red[tid + o] : red[tid];
        __syncthreads();
    }
    mx = red[0];
    // 2. e_t (each score was written by thread 2 (t % TC) of its chunk)
    for (int t0 = 0; t0 < seq; t0 += TC) {
        const int t = t0 + r;
        if (r < min(TC, seq - t0) && hf == 0) sc[t] = expf_tg(sc[t] - mx);
    }
    __syncthreads();
    // 3. sum in order, 1024 values at a time through LDS
    float sum = 0.0f;
    for (int t0 = 0; t0 < seq; t0 += 1024) {
        const int n = min(1024, seq - t0);
        for (int i = tid; i < n; i += 256) wl[i] = sc[t0 + i];
        __syncthreads();
        if (tid == 0) {
#pragma unroll 16
            for (int i = 0; i < n; i++) sum = sum + wl[i];
        }
        __syncthreads();
    }
    if (tid == 0) inv_sum = 1.0f / sum;
    __syncthreads();
    const float is = inv_sum;
    // 4. weighted values: chunks of TC rows of V and their weights in LDS
    float o0 = 0.0f, o1 = 0.0f;  // elements tid and tid + 256
    for (int t0 = 0; t0 < seq; t0 += TC) {
        const int n = min(TC, seq - t0);
        att_stage(lds, hd, vch + (size_t)t0 * hd, n, hd);
        for (int i = tid; i < n; i += 256) wl[i] = sc[t0 + i] * is;
        __syncthreads();
#pragma unroll 8
        for (int t = 0; t < n; t++) {
            const float w = wl[t];
            const float *vt = lds + t * hd;
            if (tid < hd4)
                o0 = __builtin_fmaf(w, vt[tid], o0);
            else if (tid < hd)
                o0 = o0 + w * vt[tid];
            if (tid + 256 < hd4)
                o1 = __builtin_fmaf(w, vt[tid + 256], o1);
            else if (tid + 256 < hd)
                o1 = o1 + w * vt[tid + 256];
        }
        __syncthreads();
    }
    if (tid < hd) out[(size_t)h * hd + tid] = o0;
    if (tid + 256 < hd) out[(size_t)h * hd + tid + 256] = o1;
}

// x[i] += a[i] (libtinygiant.c:682,700)
__global__ __launch_bounds__(256) void k_add_vec(float *__restrict__ x, const float *__restrict__ a, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = x[i] + a[i];
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
    TG_LAUNCH(k_matmul_q4k, dim3(lg_cdiv(nrows, 4)), dim3(256), 0, st, W, static_cast<const Q8K *>(xq), y,
                       nrows, bpr);
    return hipGetLastError();
}

hipError_t launch_matmul_q6k(const uint8_t *W, const void *xq, float *y, int nrows, int bpr, hipStream_t st) {
    if (nrows <= 0) return hipSuccess;
    TG_LAUNCH(k_matmul_q6k, dim3(lg_cdiv(nrows, 4)), dim3(256), 0, st, W, static_cast<const Q8K *>(xq), y,
                       nrows, bpr);
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

hipError_t launch_attn_heads(const float *q, const float *kc, const float *vc, float *scr, float *out, int n_heads,
                             int seq, int hd, int ratio, float inv_sqrt, hipStream_t st) {
    if (hd > 512 || hd < 2 || n_heads <= 0) return hipErrorInvalidValue;
    static bool lds_set = false;  // the largest chunk (any hd) fits 70 KB of dynamic LDS
    if (!lds_set) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_attn_head, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 72 * 1024);
        if (e != hipSuccess) return e;
        lds_set = true;
    }
    TG_LAUNCH(k_attn_head, dim3(n_heads), dim3(256), att_lds_bytes(hd), st, q, kc, vc, scr, out, seq, hd, ratio,
              inv_sqrt);
    return hipGetLastError();
}

hipError_t launch_add_vec(float *x, const float *a, int n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    TG_LAUNCH(k_add_vec, dim3(lg_cdiv(n, 256)), dim3(256), 0, st, x, a, n);
    return hipGetLastError();
}

hipError_t launch_acc_scaled(float *out, const float *v, float w, int n, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    TG_LAUNCH(k_acc_scaled, dim3(lg_cdiv(n, 256)), dim3(256), 0, st, out, v, w, n);
    return hipGetLastError();
}

}  // namespace tg
