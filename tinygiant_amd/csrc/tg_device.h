// tg_device.h -- device helpers for the gfx950 MoE expert kernels.
//
// Numerics contract: every floating-point step below is written out (fmaf
// where fused, nothing else contracted: the library is compiled with
// -ffp-contract=off and correctly rounded fp32 divide/sqrt), so each kernel
// rounds exactly as the host definition of the same step does.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define TG_DEV __device__ __forceinline__

namespace tg {

constexpr int QK = 32;          // values per Q4_0 / Q8_0 block
constexpr int Q40_BYTES = 18;   // {half d; u8 qs[16]}
constexpr int Q80_BYTES = 34;   // {half d; i8 qs[32]}
constexpr int WAVE = 64;

// ---------------------------------------------------------------- halves
TG_DEV float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// LDS written by some lanes of a wave and read by others of the same wave:
// a wave's LDS operations complete in order; this keeps the compiler from
// reordering them across the hand-off
TG_DEV void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// round to nearest even (v_cvt_f16_f32 in the default mode)
TG_DEV uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// ---------------------------------------------------------------- exp
// exp(x): Cody-Waite reduction x = n ln2 + r with a 15-bit head of ln2 (so
// n * head is exact), e^r by the degree-7 Taylor polynomial in Horner form,
// result scaled by 2^n.  Arguments are clamped to [-87, 88] so the result
// is always a finite normal float.
TG_DEV float expf_tg(float x) {
    x = x > 88.0f ? 88.0f : x;
    x = x < -87.0f ? -87.0f : x;
    float n = __builtin_rintf(x * 1.44269502f);
    float r = __builtin_fmaf(n, -0.693145751953125f, x);
    r = __builtin_fmaf(n, -1.42860677e-06f, r);
    float p = 1.98412698e-04f;
    p = __builtin_fmaf(p, r, 1.38888889e-03f);
    p = __builtin_fmaf(p, r, 8.33333333e-03f);
    p = __builtin_fmaf(p, r, 4.16666667e-02f);
    p = __builtin_fmaf(p, r, 1.66666667e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)n);
}

// SiLU(g) * u = g / (1 + e^-g) * u (libtinygiant.c:580-583).
TG_DEV float silu_mul(float g, float u) {
    float e = expf_tg(-g);
    float s = g / (1.0f + e);
    return s * u;
}

// ---------------------------------------------------------------- RNG
// SplitMix64 finaliser (Steele, Lea & Flood 2014) on counters; one N(0,1)
// draw per counter by Box-Muller with float32 series for ln and cos.
TG_DEV uint64_t splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

TG_DEV uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return splitmix64(seed ^ splitmix64(stream ^ 0x6A09E667F3BCC909ull));
}

TG_DEV float ln_unit(float u) {
    uint32_t b = __float_as_uint(u);
    int e = (int)((b >> 23) & 0xFFu) - 127;
    float m = __uint_as_float((b & 0x7FFFFFu) | 0x3F800000u);
    if (m > 1.41421356f) { m = m * 0.5f; e = e + 1; }
    float f = m - 1.0f;
    float s = f / (2.0f + f);
    float z = s * s;
    float p = 0.0909090909f;
    p = __builtin_fmaf(p, z, 0.111111111f);
    p = __builtin_fmaf(p, z, 0.142857143f);
    p = __builtin_fmaf(p, z, 0.2f);
    p = __builtin_fmaf(p, z, 0.333333333f);
    p = __builtin_fmaf(p, z, 1.0f);
    float lnm = (2.0f * s) * p;
    return __builtin_fmaf((float)e, 0.693147182f, lnm);
}

TG_DEV float cos2pi(float u) {
    int q = (int)(u * 4.0f);
    q = q > 3 ? 3 : q;
    float r = u - 0.25f * (float)q;
    float t = r * 6.28318531f;
    float z = t * t;
    float c = -1.14707456e-11f;
    c = __builtin_fmaf(c, z, 2.08767570e-09f);
    c = __builtin_fmaf(c, z, -2.75573192e-07f);
    c = __builtin_fmaf(c, z, 2.48015873e-05f);
    c = __builtin_fmaf(c, z, -1.38888889e-03f);
    c = __builtin_fmaf(c, z, 4.16666667e-02f);
    c = __builtin_fmaf(c, z, -0.5f);
    c = __builtin_fmaf(c, z, 1.0f);
    float s = -7.64716373e-13f;
    s = __builtin_fmaf(s, z, 1.60590438e-10f);
    s = __builtin_fmaf(s, z, -2.50521084e-08f);
    s = __builtin_fmaf(s, z, 2.75573192e-06f);
    s = __builtin_fmaf(s, z, -1.98412698e-04f);
    s = __builtin_fmaf(s, z, 8.33333333e-03f);
    s = __builtin_fmaf(s, z, -1.66666667e-01f);
    s = s * z;
    s = __builtin_fmaf(s, t, t);
    return q == 0 ? c : (q == 1 ? -s : (q == 2 ? -c : s));
}

TG_DEV float normal_at(uint64_t key, uint64_t index) {
    uint64_t b = splitmix64(key + index * 0xD1B54A32D192ED03ull);
    float u1 = (float)((uint32_t)(b >> 40) + 1u) * 5.96046448e-08f;
    float u2 = (float)((uint32_t)(b >> 16) & 0xFFFFFFu) * 5.96046448e-08f;
    float rad = __builtin_sqrtf(-2.0f * ln_unit(u1));
    return rad * cos2pi(u2);
}

// ---------------------------------------------------------------- waves
TG_DEV float wave_sum(float v) {
    // xor butterfly 32..1: every lane ends with the same, order-fixed sum
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) v = v + __shfl_xor(v, s, WAVE);
    return v;
}

// Sum of x[0..n) squared over a 256-thread block: lane t accumulates float4
// chunks t, t+256, ... with fma, xor-butterfly inside each wave, then
// (w0 + w1) + (w2 + w3).  red: 4 floats of LDS.  Requires blockDim.x == 256.
TG_DEV float block_sumsq(const float *__restrict__ x, int n, float *red) {
    const int tid = threadIdx.x;
    float a = 0.0f;
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    for (int q = tid; q < n / 4; q += 256) {
        float4 v = x4[q];
        a = __builtin_fmaf(v.x, v.x, a);
        a = __builtin_fmaf(v.y, v.y, a);
        a = __builtin_fmaf(v.z, v.z, a);
        a = __builtin_fmaf(v.w, v.w, a);
    }
    a = wave_sum(a);
    if ((tid & 63) == 0) red[tid >> 6] = a;
    __syncthreads();
    float tot = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return tot;
}

// s_waitcnt immediate (gfx9 encoding) that waits for all vector memory
// operations of the wave and for nothing else (expcnt 7, lgkmcnt 15)
constexpr int VMCNT0 = (7 << 4) | (15 << 8);

// v through an empty asm at the point of use: a conversion of a loaded value
// (fp16 scale to float) stays there instead of being hoisted next to its
// load, where it would make the wave wait for the load early.
TG_DEV uint32_t at_use(uint32_t v) {
    __asm__ volatile("" : "+v"(v));
    return v;
}

// Workgroup barrier that orders LDS only (waits for this wave's LDS
// operations, not for its global loads): weight loads issued before it stay
// in flight across it.  For barriers whose data is all in LDS.
TG_DEV void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

typedef __attribute__((address_space(3))) uint8_t lds_u8;
TG_DEV uint32_t lds_addr(uint8_t *smem, int off) { return (uint32_t)(uintptr_t)(lds_u8 *)(smem + off); }
// global -> LDS without registers: lane l's 16 (4) bytes land at LDS byte
// address m0 + 16 l (4 l); m0 must be the same on every lane.  Written as the bare instructions so the
// compiler's wait insertion does not treat them as writes it must wait for
// before every later LDS read (it cannot tell the staged buffers apart from
// the ones being read); the kernel waits for them itself (vmcnt, then a
// barrier when other waves read them) before reading what they wrote.  The
// compiler does not count them either: its own vmcnt waits stay correct
// (a younger load in flight only makes a wait stricter), and a wait of
// its for a load issued after them covers them, since loads retire in order.
TG_DEV void lds_dma16(const void *src, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src),
                 "s"(__builtin_amdgcn_readfirstlane(m0)) : "memory", "m0");
}
TG_DEV void lds_dma4(const void *src, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(src),
                 "s"(__builtin_amdgcn_readfirstlane(m0)) : "memory", "m0");
}
// The same at agent scope (sc1): the bytes come from the device's point of
// coherence, not from a copy an XCD's L2 may still hold, for data another
// block of the same launch wrote with agent-scope stores.
TG_DEV void lds_dma16_coh(const void *src, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off sc1" ::"v"(src),
                 "s"(__builtin_amdgcn_readfirstlane(m0)) : "memory", "m0");
}
TG_DEV void lds_dma4_coh(const void *src, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off sc1" ::"v"(src),
                 "s"(__builtin_amdgcn_readfirstlane(m0)) : "memory", "m0");
}

// Tagged words: a 32-bit payload and a 32-bit tag in one 64-bit word,
// stored and loaded with relaxed agent-scope atomics, so a reader that sees
// the tag it expects also sees the payload stored with it.
TG_DEV void ll_put(uint64_t *p, uint32_t v, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | (uint64_t)v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

TG_DEV uint64_t ll_get(const uint64_t *p) {
    return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

TG_DEV float rms_scale(float ss, int n, float eps) {
    return 1.0f / __builtin_sqrtf(ss / (float)n + eps);
}

// Q8_0 of the value held by this lane, lanes grouped by 32 (a block):
// amax over the group, d = amax / 127, q = rne(v * 127 / amax).  Returns q;
// dscale = float(half(d)) (the scale the dot products use) and qsum = sum of
// the group's q.  All 64 lanes must call it.
TG_DEV int q8_lane(float v, float &dscale, int &qsum, uint16_t &dhalf) {
    float a = fabsf(v);
#pragma unroll
    for (int s = 16; s >= 1; s >>= 1) {
        float o = __shfl_xor(a, s, WAVE);
        a = o > a ? o : a;
    }
    float d = a / 127.0f;
    float inv = a > 0.0f ? 127.0f / a : 0.0f;
    int q = (int)__builtin_rintf(v * inv);
    int sum = q;
#pragma unroll
    for (int s = 16; s >= 1; s >>= 1) sum += __shfl_xor(sum, s, WAVE);
    dhalf = f2h(d);
    dscale = h2f(dhalf);
    qsum = sum;
    return q;
}

// sum_i q_w,i * q_x,i over one block: w = the block's 16 nibble bytes
// (element j < 16 in the low nibble of byte j, element j+16 in the high
// nibble), x = its 32 activation bytes as 8 dwords.  Nibbles 0..15 are
// valid signed bytes, so the signed 4-way dot applies.
TG_DEV int dot_q4_q8(uint4 w, const int *x) {
    const uint32_t m = 0x0F0F0F0Fu;
    int s = 0;
    s = __builtin_amdgcn_sdot4((int)(w.x & m), x[0], s, false);
    s = __builtin_amdgcn_sdot4((int)(w.y & m), x[1], s, false);
    s = __builtin_amdgcn_sdot4((int)(w.z & m), x[2], s, false);
    s = __builtin_amdgcn_sdot4((int)(w.w & m), x[3], s, false);
    s = __builtin_amdgcn_sdot4((int)((w.x >> 4) & m), x[4], s, false);
    s = __builtin_amdgcn_sdot4((int)((w.y >> 4) & m), x[5], s, false);
    s = __builtin_amdgcn_sdot4((int)((w.z >> 4) & m), x[6], s, false);
    s = __builtin_amdgcn_sdot4((int)((w.w >> 4) & m), x[7], s, false);
    return s;
}

// numpy's pairwise float32 sum for n <= 64 (n < 8: sequential from 0).
TG_DEV float np_pairwise_sum(const float *a, int n) {
    if (n < 8) {
        float r = 0.0f;
        for (int i = 0; i < n; i++) r = r + a[i];
        return r;
    }
    float r0 = a[0], r1 = a[1], r2 = a[2], r3 = a[3], r4 = a[4], r5 = a[5], r6 = a[6], r7 = a[7];
    int i;
    for (i = 8; i < n - (n % 8); i += 8) {
        r0 = r0 + a[i]; r1 = r1 + a[i + 1]; r2 = r2 + a[i + 2]; r3 = r3 + a[i + 3];
        r4 = r4 + a[i + 4]; r5 = r5 + a[i + 5]; r6 = r6 + a[i + 6]; r7 = r7 + a[i + 7];
    }
    float res = ((r0 + r1) + (r2 + r3)) + ((r4 + r5) + (r6 + r7));
    for (; i < n; i++) res = res + a[i];
    return res;
}

}  // namespace tg
