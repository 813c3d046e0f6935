// tg_mfma.hip -- grouped-expert GEMM on int8 MFMA (batched decode, prefill).
//
// Work item = (expert e, up to MT*32 entries of its group).  A block of four
// waves shares the item's activations, staged through LDS in chunks of
// MF_KC Q4_0 blocks (double-buffered, loaded by all 256 threads); each wave
// owns one tile of 32 weight rows and walks its Q4_0 blocks b.  Per block and
// tile of 32 entries, one v_mfma_i32_32x32x32_i8 computes the block's 32 x 32
// integer dot products exactly; K = 32 is one Q4_0 / Q8_0 block.
//
// Operands (lane l, half h = l / 32; A lane h*32+m byte j pairs with B lane
// h*32+n byte j, measured on gfx950):
//   A  q - 8 of weight row m = l % 32, block b, elements 16h .. 16h+15 (the
//      low (h = 0) or high (h = 1) nibbles of the row's 16 bytes) as int8,
//      from byte-wise (q | 0x80) - 8 ^ 0x80, which never borrows across bytes
//   B  Q8_0 values of entry n = l % 32 of the tile, block b, elements
//      16h .. 16h+15 (one 128-bit LDS read)
//   C  0x4B400000 for every element
// so D = 0x4B400000 + S with S = sum (q_w - 8) q_x, |S| <= 32512: D's bits
// are the float 1.5 * 2^23 + S exactly.  Output layout: lane l, register r
// holds (weight row m, entry n) = (8 (r/4) + 4h + r%4, l % 32).
//
// Epilogue per block (the row-dot definition, bit for bit):
//   u   = fma(float_bits(D), dw_m, -1.5 * 2^23 * dw_m)   = round(S * dw_m)
//         (the constant is exact: dw is a half)
//   acc = fma(u, dx_n, acc)
// dx_n is one value per lane; the 16 row scales dw_m a lane needs, and
// their -1.5 * 2^23 multiples, are read from a per-wave LDS table kept in
// register order, shared by the M-tiles.  M-tiles past the item's last
// entry are skipped (the loop is compiled once per active-tile count).
// Gate/up then applies SwiGLU and Q8_0 per (entry, 32 rows): the 32 values
// of one entry sit in lanes n and n + 32, 16 registers each.  Down writes
// fp32 rows per entry for the combine.
#include <atomic>

#include "tg_device.h"
#include "tg_internal.h"

namespace tg {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

template <int N> struct Tiles { static constexpr int value = N; };

// Q4_0 blocks of A prefetched ahead per wave: deeper where a block holds
// one M-tile (little work per weight byte, the stream is latency-bound)
__host__ __device__ constexpr int mf_pf(int mt) { return mt == 1 ? 8 : 4; }
constexpr int MF_KC = 8;               // Q4_0 blocks per staged activation chunk
constexpr int MF_TS = MF_KC * 32 + 16;  // LDS bytes per staged activation row (16 pad)
constexpr uint32_t MAGIC_I = 0x4B400000u;
constexpr float MAGIC_F = 12582912.0f;  // 1.5 * 2^23

// nibble bytes (0..15 each) -> q - 8 as int8 per byte
TG_DEV int nib_s8(uint32_t nb4) { return (int)(((nb4 | 0x80808080u) - 0x08080808u) ^ 0x80808080u); }

TG_DEV v4i nib_lo(uint4 w) {
    v4i r;
    r.x = nib_s8(w.x & 0x0F0F0F0Fu); r.y = nib_s8(w.y & 0x0F0F0F0Fu);
    r.z = nib_s8(w.z & 0x0F0F0F0Fu); r.w = nib_s8(w.w & 0x0F0F0F0Fu);
    return r;
}

TG_DEV v4i nib_hi(uint4 w) {
    v4i r;
    r.x = nib_s8((w.x >> 4) & 0x0F0F0F0Fu); r.y = nib_s8((w.y >> 4) & 0x0F0F0F0Fu);
    r.z = nib_s8((w.z >> 4) & 0x0F0F0F0Fu); r.w = nib_s8((w.w >> 4) & 0x0F0F0F0Fu);
    return r;
}

// LDS: two chunk buffers of [M rows][MF_TS bytes] activations and
// [MF_KC][M] activation scales, then per wave two [MF_KC][2][2][16] tables
// of weight scales (per half: 16 dw, then their -1.5 * 2^23 multiples).
// Gate/up's hand-off of the up sums (NW/2 tiles x MT x 16 registers x 64
// lanes) reuses the activation buffers after the block loop.
__host__ __device__ inline size_t mf_lds_bytes(int mt, int nw) {
    const size_t m = 32 * (size_t)mt;
    return 2 * m * MF_TS + 2 * MF_KC * m * 4 + (size_t)nw * 2 * MF_KC * 64 * 4;
}

// waves per block: 8 at four M-tiles (two waves per SIMD share one staged
// activation tile), else 4
__host__ __device__ constexpr int mf_waves(int mt) { return mt >= 4 ? 8 : 4; }

// PAIR: gate/up.  Waves 2i / 2i+1 of a block take gate / up of tile
// (NW/2) x + i; after the block loop the up waves hand their sums to the
// gate waves through LDS, which apply SwiGLU and Q8_0 and write h.
// Otherwise down: NW tiles of down rows per block, fp32 rows out.
// Activations are indexed by token (entry / k) for gate/up and by entry for
// down.
template <int MT, bool PAIR, int NW = mf_waves(MT)>
__global__ __launch_bounds__(NW * 64) void k_mfma_grouped(const uint8_t *__restrict__ layer_pl, Shape s,
                                                             const int32_t *__restrict__ work,
                                                             const int32_t *__restrict__ work_n,
                                                             const int32_t *__restrict__ entries,
                                                             const int8_t *__restrict__ aq,
                                                             const float *__restrict__ ad, int8_t *__restrict__ oq,
                                                             float *__restrict__ od, int *__restrict__ os,
                                                             float *__restrict__ D) {
    constexpr int M = MT * 32;
    constexpr int NT = NW * 64;                      // threads per block
    constexpr int TP = 2 * MF_KC;                    // 16-byte pieces per row and chunk
    constexpr int NTP = M * TP / NT;                 // pieces staged per thread
    constexpr int NDX = M * MF_KC / NT;              // activation scales staged per thread
    constexpr int MF_PF = mf_pf(MT);
    static_assert(NT % TP == 0 && NT % MF_KC == 0 && MF_KC % MF_PF == 0, "staging map");
    static_assert(NTP >= 1 && NDX >= 1 && (M * TP) % NT == 0 && (M * MF_KC) % NT == 0, "staging map");
    extern __shared__ __align__(16) uint8_t smem[];
    const int wi = blockIdx.y;
    if (wi >= work_n[0]) return;  // uniform over the block
    const int e = work[3 * wi], o = work[3 * wi + 1], c = work[3 * wi + 2];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 31, h = lane >> 5;
    const int K = PAIR ? s.H : s.I, nb = K / QK, rows = PAIR ? s.I : s.H, k = s.k;
    const int nch = (nb + MF_KC - 1) / MF_KC;

    uint8_t *tokl = smem;                                                     // [2][M][MF_TS]
    float *dxl = reinterpret_cast<float *>(smem + 2 * M * MF_TS);             // [2][MF_KC][M]
    float *dwl = dxl + 2 * MF_KC * M + wave * (2 * MF_KC * 64);               // [2][MF_KC][2][2][16]

    // staging map: piece p of row t = tid / TP + u * (NT / TP); scale of
    // block tid % MF_KC of row tid / MF_KC + u * (NT / MF_KC)
    const int sp = tid % TP, sb = tid % MF_KC;
    int toff[NTP], doff[NDX];
#pragma unroll
    for (int u = 0; u < NTP; u++) {
        const int t = tid / TP + u * (NT / TP);
        toff[u] = -1;
        if (t < c) {
            const int ent = entries[o + t];
            toff[u] = (PAIR ? ent / k : ent) * K;
        }
    }
#pragma unroll
    for (int u = 0; u < NDX; u++) {
        const int t = tid / MF_KC + u * (NT / MF_KC);
        doff[u] = -1;
        if (t < c) {
            const int ent = entries[o + t];
            doff[u] = (PAIR ? ent / k : ent) * nb;
        }
    }

    // this wave's weight tile; an out-of-range tile computes on row n and
    // stores nothing
    const int mat = PAIR ? (wave & 1) : 0;  // 0 gate / down, 1 up
    const int nt = PAIR ? blockIdx.x * (NW / 2) + (wave >> 1) : blockIdx.x * NW + wave;
    const bool valid = nt * 32 < rows;
    const int R = valid ? nt * 32 + n : n;
    const uint8_t *ex = layer_pl + (size_t)e * s.EB;
    const uint8_t *tb = PAIR ? ex + (size_t)mat * s.GB : ex + 2 * s.GB;
    const size_t ntb = (size_t)rows * nb;
    const uint4 *q0 = reinterpret_cast<const uint4 *>(tb) + (size_t)R * nb;
    const uint16_t *s0 = reinterpret_cast<const uint16_t *>(tb + ntb * 16) + (size_t)R * nb;
    // slot of row n in the register-ordered scale table: half (n / 4) % 2,
    // register 4 (n / 8) + n % 4; its -1.5 * 2^23 multiple 16 slots on
    const int wslot = ((n >> 2) & 1) * 32 + 4 * (n >> 3) + (n & 3);

    uint4 sv[NTP];
    float sd[NDX];
    uint16_t ws[MF_KC];
    auto stage = [&](int ch) {
#pragma unroll
        for (int u = 0; u < NTP; u++) {
            const int kb = ch * MF_KC * 32 + sp * 16;
            sv[u] = make_uint4(0u, 0u, 0u, 0u);
            if (toff[u] >= 0 && kb < K) sv[u] = *reinterpret_cast<const uint4 *>(aq + toff[u] + kb);
        }
#pragma unroll
        for (int u = 0; u < NDX; u++) {
            const int b = ch * MF_KC + sb;
            sd[u] = (doff[u] >= 0 && b < nb) ? ad[doff[u] + b] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < MF_KC; j++) {
            const int b = ch * MF_KC + j;
            ws[j] = (h == 0 && b < nb) ? s0[b] : (uint16_t)0;
        }
    };
    auto commit = [&](int q) {
#pragma unroll
        for (int u = 0; u < NTP; u++) {
            const int t = tid / TP + u * (NT / TP);
            *reinterpret_cast<uint4 *>(tokl + ((size_t)q * M + t) * MF_TS + sp * 16) = sv[u];
        }
#pragma unroll
        for (int u = 0; u < NDX; u++) {
            const int t = tid / MF_KC + u * (NT / MF_KC);
            dxl[(q * MF_KC + sb) * M + t] = sd[u];
        }
        if (h == 0) {
#pragma unroll
            for (int j = 0; j < MF_KC; j++) {
                const float d = h2f(ws[j]);
                dwl[(q * MF_KC + j) * 64 + wslot] = d;
                dwl[(q * MF_KC + j) * 64 + wslot + 16] = -MAGIC_F * d;
            }
        }
    };

    float acc[MT][16];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[mt][r] = 0.0f;

    stage(0);
    commit(0);
    // A prefetch ring: block b sits in slot b % MF_PF
    uint4 w0[MF_PF];
#pragma unroll
    for (int p = 0; p < MF_PF; p++)
        if (p < nb) w0[p] = q0[p];
    v16i cmag;
#pragma unroll
    for (int r = 0; r < 16; r++) cmag[r] = (int)MAGIC_I;
    __syncthreads();

    // The block loop runs the item's active M-tiles only (tiles at or past
    // c hold no entries); `na` is their count as a compile-time constant.
    auto run = [&](auto na) {
        constexpr int NA = decltype(na)::value;
        for (int ch = 0; ch < nch; ch++) {
            const int q = ch & 1;
            if (ch + 1 < nch) stage(ch + 1);
            const uint8_t *tq = tokl + (size_t)q * M * MF_TS + (size_t)n * MF_TS + 16 * h;
            const float *xq = dxl + q * MF_KC * M + n;
            const float *wq = dwl + q * MF_KC * 64 + 32 * h;
#pragma unroll
            for (int bl = 0; bl < MF_KC; bl++) {
                const int b = ch * MF_KC + bl;
                if (b < nb) {
                    const v4i wa = h ? nib_hi(w0[bl % MF_PF]) : nib_lo(w0[bl % MF_PF]);
                    if (b + MF_PF < nb) w0[bl % MF_PF] = q0[b + MF_PF];
                    v4i tbv[NA];
                    float dx[NA];
#pragma unroll
                    for (int mt = 0; mt < NA; mt++) {
                        tbv[mt] = *reinterpret_cast<const v4i *>(tq + (size_t)mt * 32 * MF_TS + bl * 32);
                        dx[mt] = xq[bl * M + mt * 32];
                    }
                    float dw[16], cw[16];
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const float4 v = *reinterpret_cast<const float4 *>(wq + bl * 64 + 4 * g);
                        dw[4 * g] = v.x; dw[4 * g + 1] = v.y; dw[4 * g + 2] = v.z; dw[4 * g + 3] = v.w;
                        const float4 u = *reinterpret_cast<const float4 *>(wq + bl * 64 + 16 + 4 * g);
                        cw[4 * g] = u.x; cw[4 * g + 1] = u.y; cw[4 * g + 2] = u.z; cw[4 * g + 3] = u.w;
                    }
                    // tile mt + 1's MFMA is issued before tile mt's epilogue:
                    // two result sets live at a time, which keeps them in VGPRs
                    v16i rc = __builtin_amdgcn_mfma_i32_32x32x32_i8(wa, tbv[0], cmag, 0, 0, 0);
#pragma unroll
                    for (int mt = 0; mt < NA; mt++) {
                        v16i rn;
                        if (mt + 1 < NA) rn = __builtin_amdgcn_mfma_i32_32x32x32_i8(wa, tbv[mt + 1], cmag, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const float u = __builtin_fmaf(__int_as_float(rc[r]), dw[r], cw[r]);
                            acc[mt][r] = __builtin_fmaf(u, dx[mt], acc[mt][r]);
                        }
                        if (mt + 1 < NA) rc = rn;
                    }
                }
            }
            if (ch + 1 < nch) commit(q ^ 1);
            __syncthreads();
        }
    };
    // (a three-tile variant spills registers: three active tiles run as four)
    const int na = (c + 31) >> 5;
    if constexpr (MT >= 4) {
        if (na >= 3) run(Tiles<4>{});
        else if (na == 2) run(Tiles<2>{});
        else run(Tiles<1>{});
    } else if constexpr (MT == 2) {
        if (na >= 2) run(Tiles<2>{});
        else run(Tiles<1>{});
    } else {
        run(Tiles<1>{});
    }

    if (PAIR) {
        // up sums -> LDS (over the activation buffers), gate waves combine
        float *x = reinterpret_cast<float *>(smem) + (size_t)(wave >> 1) * MT * 16 * 64;
        if (mat == 1) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int r = 0; r < 16; r++) x[(mt * 16 + r) * 64 + lane] = acc[mt][r];
        }
        __syncthreads();
        if (mat == 1) return;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int t = mt * 32 + n;
            const bool on = valid && t < c;
            // SwiGLU, then Q8_0 over the entry's 32 rows (16 here, 16 in lane ^ 32)
            float hv[16], a = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                hv[r] = on ? silu_mul(acc[mt][r], x[(mt * 16 + r) * 64 + lane]) : 0.0f;
                const float v = fabsf(hv[r]);
                a = v > a ? v : a;
            }
            const float ao = __shfl_xor(a, 32, WAVE);
            a = ao > a ? ao : a;
            const float d = a / 127.0f;
            const float inv = a > 0.0f ? 127.0f / a : 0.0f;
            int qv[16], sum = 0;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                qv[r] = (int)__builtin_rintf(hv[r] * inv);
                sum += qv[r];
            }
            sum += __shfl_xor(sum, 32, WAVE);
            if (on) {
                const int ent = entries[o + t];
                int8_t *dst = oq + (size_t)ent * s.I + nt * 32 + 4 * h;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t w = (uint32_t)(qv[4 * j] & 0xFF) | ((uint32_t)(qv[4 * j + 1] & 0xFF) << 8) |
                                       ((uint32_t)(qv[4 * j + 2] & 0xFF) << 16) |
                                       ((uint32_t)(qv[4 * j + 3] & 0xFF) << 24);
                    *reinterpret_cast<uint32_t *>(dst + 8 * j) = w;
                }
                if (h == 0) {
                    od[(size_t)ent * s.nbI + nt] = h2f(f2h(d));
                    os[(size_t)ent * s.nbI + nt] = sum;
                }
            }
        }
    } else if (valid) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int t = mt * 32 + n;
            if (t < c) {
                float *dst = D + (size_t)entries[o + t] * s.H + nt * 32 + 4 * h;
#pragma unroll
                for (int j = 0; j < 4; j++)
                    *reinterpret_cast<float4 *>(dst + 8 * j) =
                        make_float4(acc[mt][4 * j], acc[mt][4 * j + 1], acc[mt][4 * j + 2], acc[mt][4 * j + 3]);
            }
        }
    }
}

// ================================================================ combine in the down launch
// The weighted combine of the grouped path (engine.py:240-258: out = x +
// sum_j w_j down_j; the slots in order k-1 .. 0 from zero, then the
// residual, as k_combine) inside the down launch.  A block stores its D rows
// with device-coherent stores, waits until every one of them is
// acknowledged, and then counts each of its entries in at (token, tile of
// FC_ROWS rows).  The block whose count reaches k holds the last of that
// token's k slots over its tile: it folds the k rows there (coherent loads)
// and writes the output rows, and sets the count back to zero for the next
// call.  No block waits for another, so the launch completes in any
// dispatch order.
TG_DEV void st_coh(float *p, float v) {
    __hip_atomic_store(reinterpret_cast<uint32_t *>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
TG_DEV void st_coh2(float *p, float a, float b) {  // p 8-byte aligned
    const uint64_t v = (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
    __hip_atomic_store(reinterpret_cast<uint64_t *>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
TG_DEV float ld_coh(const float *p) {
    return __uint_as_float(__hip_atomic_load(const_cast<uint32_t *>(reinterpret_cast<const uint32_t *>(p)),
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// Every thread of the block calls it after its last D store; smem: at least
// 4 (c + 1) bytes, free.  Tokens per pass: NT / FC_ROWS * FC_TOK.
constexpr int FC_TOK = 4;   // tokens per thread per pass (k loads each in flight)
template <int NT>
TG_DEV void fused_combine(const FuseArgs &F, const Shape &s, const int32_t *__restrict__ entries, int o, int c,
                          int tile, const float *D, uint8_t *smem) {
    static_assert(NT % FC_ROWS == 0, "whole rows of tokens per pass");
    constexpr int TP = NT / FC_ROWS;
    int *ln = reinterpret_cast<int *>(smem), *ltok = ln + 1;
    __builtin_amdgcn_s_waitcnt(VMCNT0);  // this thread's D stores acknowledged
    __syncthreads();                     // ... every thread's; the LDS is free
    const int tid = threadIdx.x, k = s.k, H = s.H, ntile = H / FC_ROWS;
    if (tid == 0) *ln = 0;
    __syncthreads();
    for (int t = tid; t < c; t += NT) {
        const int tok = entries[o + t] / k;
        uint32_t *p = F.cnt + (size_t)tok * ntile + tile;
        if (__hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(k - 1)) {
            __hip_atomic_store(p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ltok[atomicAdd(ln, 1)] = tok;
        }
    }
    __syncthreads();
    const int nl = *ln, r = tid % FC_ROWS, q = tid / FC_ROWS, row = tile * FC_ROWS + r;
    for (int b0 = 0; b0 < nl; b0 += TP * FC_TOK) {
        int tok[FC_TOK];
#pragma unroll
        for (int i = 0; i < FC_TOK; i++) {
            const int b = b0 + q + TP * i;
            tok[i] = ltok[b < nl ? b : nl - 1];  // past the list: the last token again, not stored
        }
        float acc[FC_TOK];
#pragma unroll
        for (int i = 0; i < FC_TOK; i++) acc[i] = 0.0f;
        for (int j0 = k - 1; j0 >= 0; j0 -= 8) {  // slots j0 .. j0 - 7, loads of every token in flight
            float v[FC_TOK][8];
#pragma unroll
            for (int i = 0; i < FC_TOK; i++)
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const int j = j0 - u >= 0 ? j0 - u : 0;
                    v[i][u] = ld_coh(D + ((size_t)tok[i] * k + j) * H + row);
                }
#pragma unroll
            for (int i = 0; i < FC_TOK; i++)
#pragma unroll
                for (int u = 0; u < 8; u++)
                    if (j0 - u >= 0) acc[i] = __builtin_fmaf(F.w[(size_t)tok[i] * k + j0 - u], v[i][u], acc[i]);
        }
#pragma unroll
        for (int i = 0; i < FC_TOK; i++) {
            if (b0 + q + TP * i < nl) {
                const size_t oi = (size_t)tok[i] * H + row;
                F.out[oi] = F.resid ? F.resid[oi] + acc[i] : acc[i];
            }
        }
    }
}

// ================================================================ one M-tile
// Work items of at most 32 entries (batched decode, a few entries per expert):
// the operands swap roles, A = the item's Q8_0 activations (lane h*32+m:
// entry m, elements 16h .. 16h+15 of the block) and B = the weight nibbles
// (lane h*32+n: weight row n), so lane l, register r of the result holds
// (entry 8 (r/4) + 4h + r%4, weight row l % 32).  The weight scale is then one
// value per lane, and the epilogue runs only the register groups (8 entries
// each) that hold entries of the item.  The weight bytes enter the MFMA as
// 16 (q - 8) (as in the 16 x 16 kernel) against an inline zero accumulator,
// so D = 16 S exactly; per block and entry group u16 = round(float(D) * dw)
// = 16 round(S * dw) and acc = fma(u16, dx / 16, acc) = fma(round(S * dw),
// dx, acc) bit for bit (powers of two scale exactly), blocks in ascending
// order: the row-dot definition.  Gate/up: waves 2i / 2i+1
// take gate / up of tile 2x + i, meet in LDS, and each applies SwiGLU and
// Q8_0 to half of the entries, each entry's 32 rows (one per lane of a
// half-wave: maximum and sum by row rotations and a swap of the rows).
// Weights: per chunk of MF_KC = 8 blocks, lane (n, h) loads row n's blocks
// 4h .. 4h+3 (64 contiguous bytes; the two lanes of a row cover its whole
// 128-byte line) and, with nb % 8 == 0, the row's 8 scales in one 16-byte
// load; the loads of the next two chunks are in flight while this one
// computes.  Block bl's 16 bytes reach both lanes of the row through one
// lane-half swap.
constexpr int MS_NW = 4;    // waves per block
constexpr int MS_PF = 2;    // weight chunks in flight per wave (down; gate/up one more)

__host__ __device__ inline size_t ms_lds_bytes() { return 2 * 32 * (size_t)MF_TS + 2 * MF_KC * 32 * 4; }
// Items whose K spans at most MS_FC chunks stage all of their activations
// once, before the weight loop: [chunk][entry][256 bytes, 16-byte pieces
// rotated by the entry] then [chunk][block][entry] activation scales.
constexpr int MS_FC = 8;
__host__ __device__ inline size_t ms_full_lds_bytes() { return (size_t)MS_FC * (32 * 256 + MF_KC * 32 * 4); }

// one lane-half swap: lo takes half 0's value of v on every lane, hi half 1's
// (lane i and lane i ^ 32 end with the same pair)
TG_DEV void half_split(uint32_t v, uint32_t &lo, uint32_t &hi) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    lo = r[0];
    hi = r[1];
}

template <int CTRL>
TG_DEV float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
TG_DEV int dpp_i(int v) { return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xF, 0xF, false); }
// lane ^ 16 inside each group of 32 lanes
TG_DEV float swz16_f(float v) { return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F)); }
TG_DEV int swz16_i(int v) { return __builtin_amdgcn_ds_swizzle(v, 0x401F); }

// maximum (NaN never taken) and sum over the 32 lanes of a half-wave, in
// every lane of it
TG_DEV float half_max(float a) {
    float o;
    o = dpp_f<0x121>(a); a = o > a ? o : a;  // row_ror:1
    o = dpp_f<0x122>(a); a = o > a ? o : a;  // row_ror:2
    o = dpp_f<0x124>(a); a = o > a ? o : a;  // row_ror:4
    o = dpp_f<0x128>(a); a = o > a ? o : a;  // row_ror:8
    o = swz16_f(a); a = o > a ? o : a;
    return a;
}
TG_DEV int half_sum(int v) {
    v += dpp_i<0x121>(v);
    v += dpp_i<0x122>(v);
    v += dpp_i<0x124>(v);
    v += dpp_i<0x128>(v);
    v += swz16_i(v);
    return v;
}

// One block of the one-tile kernels: item wi, row tile bx.  GD: gate/up and
// down blocks of the same launch (k_mfma_small_gd): a gate/up block stores
// h with agent-scope stores and, once they are acknowledged, counts itself in
// at rdy[wi]; a down block waits (bounded) until all `need` gate/up blocks of
// its item have, then stages h at agent scope.
template <bool PAIR, bool SCV, bool FULL, bool GD>
TG_DEV __attribute__((always_inline)) void ms_item(const uint8_t *__restrict__ layer_pl, const Shape s,
                                                   const int32_t *__restrict__ work,
                                                   const int32_t *__restrict__ work_n,
                                                   const int32_t *__restrict__ entries,
                                                   const int8_t *__restrict__ aq, const float *__restrict__ ad,
                                                   int8_t *__restrict__ oq, float *__restrict__ od,
                                                   int *__restrict__ os, float *__restrict__ D, const FuseArgs F,
                                                   int wi, int bx, const GdArgs G) {
    // the launch's dynamic LDS, named here so its addresses stay LDS
    // addresses (through a generic pointer each cast to LDS adds a null test)
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int M = 32, NW = MS_NW, NT = NW * 64, TP = 2 * MF_KC;
    constexpr int NTP = M * TP / NT, NDX = M * MF_KC / NT;
    static_assert(NT % TP == 0 && NT % MF_KC == 0 && MF_KC == 8 && NTP >= 1 && NDX >= 1, "staging map");
    static_assert(!GD || PAIR || FULL, "a waiting down block stages its activations once, at agent scope");
    if (wi >= work_n[0]) return;  // uniform over the block
    const int e = work[3 * wi], o = work[3 * wi + 1], c = work[3 * wi + 2];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n = lane & 31, h = lane >> 5;
    const int K = PAIR ? s.H : s.I, nb = K / QK, rows = PAIR ? s.I : s.H, k = s.k;
    const int nch = (nb + MF_KC - 1) / MF_KC;

    uint8_t *tokl = smem;                                                     // [2][M][MF_TS]
    float *dxl = reinterpret_cast<float *>(smem + 2 * M * MF_TS);             // [2][MF_KC][M]

    const int sp = tid % TP, sb = tid % MF_KC;
    int toff[NTP], doff[NDX];
#pragma unroll
    for (int u = 0; u < NTP; u++) {
        const int t = tid / TP + u * (NT / TP);
        toff[u] = -1;
        if (t < c) toff[u] = (PAIR ? entries[o + t] / k : entries[o + t]) * K;
    }
#pragma unroll
    for (int u = 0; u < NDX; u++) {
        const int t = tid / MF_KC + u * (NT / MF_KC);
        doff[u] = -1;
        if (t < c) doff[u] = (PAIR ? entries[o + t] / k : entries[o + t]) * nb;
    }

    const int mat = PAIR ? (wave & 1) : 0;  // 0 gate / down, 1 up
    const int nt = PAIR ? bx * (NW / 2) + (wave >> 1) : bx * NW + wave;
    const bool valid = nt * 32 < rows;
    const int R = valid ? nt * 32 + n : n;
    const uint8_t *ex = layer_pl + (size_t)e * s.EB;
    const uint8_t *tb = PAIR ? ex + (size_t)mat * s.GB : ex + 2 * s.GB;
    const size_t ntb = (size_t)rows * nb;
    const uint4 *q0 = reinterpret_cast<const uint4 *>(tb) + (size_t)R * nb;
    const uint16_t *s0 = reinterpret_cast<const uint16_t *>(tb + ntb * 16) + (size_t)R * nb;

    // (FULL) every chunk's activations and activation scales straight into
    // LDS, issued before any weight load: the waits of the weight loop then
    // count weight loads only.  Entries past the item stage the item's last
    // entry's bytes (their sums are never stored).
    // GD down block: every gate/up block of the item has counted in
    // (bounded; when the wait runs out the rows are stored as NaN and *err set)
    bool gd_bad = false;
    if constexpr (GD && !PAIR) {
        __shared__ int gd_flag;
        if (tid == 0) {
            uint32_t tries = 0;
            int bad = 0;
            while (__hip_atomic_load(G.rdy + wi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < G.need) {
                if (++tries >= G.spin) {
                    bad = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            gd_flag = bad;
            if (bad) __hip_atomic_store(G.err, 4u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        gd_bad = gd_flag != 0;
    }

    constexpr int FA = M * 256, FD = MF_KC * M;  // bytes of one chunk's rows, scales of one chunk
    if constexpr (FULL) {
        constexpr int JA = M * 256 / (NT * 16), JD = FD / NT;  // DMA rounds per chunk: rows, scales
        static_assert(JA * NT * 16 == M * 256 && JD * NT == FD, "staging map");
        // this lane's entries (looked up once): its row slots' and its scale slots'
        const int8_t *asrc[JA];
        const float *dsrc[JD];
#pragma unroll
        for (int j = 0; j < JA; j++) {
            const int L = (j * NW + wave) * 64 + lane;  // 16-byte slot of a chunk's rows
            const int t = L >> 4, pc = ((L & 15) - t) & 15;
            const int et = entries[o + min(t, c - 1)];
            asrc[j] = aq + (size_t)(PAIR ? et / k : et) * K + pc * 16;
        }
#pragma unroll
        for (int j = 0; j < JD; j++) {
            const int L = (j * NW + wave) * 64 + lane;  // scale slot: block L / M, entry L % M
            const int et = entries[o + min(L % M, c - 1)];
            dsrc[j] = ad + (size_t)(PAIR ? et / k : et) * nb + L / M;
        }
#pragma unroll
        for (int ch = 0; ch < MS_FC; ch++) {
            if (ch < nch) {  // uniform
#pragma unroll
                for (int j = 0; j < JA; j++) {
                    const uint32_t m0 = lds_addr(smem, ch * FA + (j * NW + wave) * 1024);
                    if constexpr (GD && !PAIR)
                        lds_dma16_coh(asrc[j] + ch * MF_KC * 32, m0);
                    else
                        lds_dma16(asrc[j] + ch * MF_KC * 32, m0);
                }
#pragma unroll
                for (int j = 0; j < JD; j++) {
                    const uint32_t m0 = lds_addr(smem, MS_FC * FA + (ch * FD + (j * NW + wave) * 64) * 4);
                    if constexpr (GD && !PAIR)
                        lds_dma4_coh(dsrc[j] + ch * MF_KC, m0);
                    else
                        lds_dma4(dsrc[j] + ch * MF_KC, m0);
                }
            }
        }
    }

    // activation staging: unconditional loads from clamped, in-bounds
    // addresses (entries past the item and blocks past K select zero when
    // committed), so the waits before the commit count exactly the loads
    // issued after them and leave the weight loads in flight
    uint4 sv[NTP];
    float sd[NDX];
    auto stage = [&](int ch) {
#pragma unroll
        for (int u = 0; u < NTP; u++) {
            const int kb = min(ch * MF_KC * 32 + sp * 16, K - 16);
            sv[u] = *reinterpret_cast<const uint4 *>(aq + max(toff[u], 0) + kb);
        }
#pragma unroll
        for (int u = 0; u < NDX; u++) sd[u] = ad[max(doff[u], 0) + min(ch * MF_KC + sb, nb - 1)];
    };
    auto commit = [&](int q, int ch) {
#pragma unroll
        for (int u = 0; u < NTP; u++) {
            const int t = tid / TP + u * (NT / TP);
            const bool ok = toff[u] >= 0 && ch * MF_KC * 32 + sp * 16 < K;
            *reinterpret_cast<uint4 *>(tokl + ((size_t)q * M + t) * MF_TS + sp * 16) =
                ok ? sv[u] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < NDX; u++) {
            const int t = tid / MF_KC + u * (NT / MF_KC);
            const bool ok = doff[u] >= 0 && ch * MF_KC + sb < nb;
            dxl[(q * MF_KC + sb) * M + t] = ok ? sd[u] * 0.0625f : 0.0f;  // dx / 16, exact
        }
    };
    // row R's weights of chunk ch: blocks 8ch + 4h + i (clamped; blocks past
    // nb are never used) and the chunk's 8 scales (packed halves); chunks
    // past the last load the last one again (unconditional loads keep the
    // waits exact)
    auto wload = [&](int ch, uint4 (&w)[4], uint4 &sc) {
#pragma unroll
        for (int i = 0; i < 4; i++) w[i] = q0[min(ch * MF_KC + 4 * h + i, nb - 1)];
        if (SCV) {
            sc = *reinterpret_cast<const uint4 *>(s0 + min(ch, nch - 1) * MF_KC);
        } else {
            uint32_t hv[MF_KC];
#pragma unroll
            for (int j = 0; j < MF_KC; j++) hv[j] = s0[min(ch * MF_KC + j, nb - 1)];
            sc = make_uint4(hv[0] | hv[1] << 16, hv[2] | hv[3] << 16, hv[4] | hv[5] << 16, hv[6] | hv[7] << 16);
        }
    };

    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;

    // weights run PF chunks ahead in PF + 1 register sets, each with a
    // fixed role per unrolled step (a copy between sets would wait for the
    // loads in flight); the activations one chunk ahead, issued before the
    // newer weight loads so the wait before their commit leaves those in
    // flight
    // (gate / up with 16-byte scale loads: three chunks ahead in four sets,
    // still two waves per SIMD; otherwise two ahead in three: the down
    // launch measured slower with three, 80.5 -> 94.9 us at H 4096, I 1536)
    constexpr int PF = PAIR && SCV ? MS_PF + 1 : MS_PF;
    static_assert(MS_PF == 2, "three or four register sets");
    uint4 wa[4], sa, wb[4], sbv, wcx[4], scx, wdx[4], sdx;
    wload(0, wa, sa);
    if constexpr (!FULL) stage(0);
    wload(1, wb, sbv);
    if constexpr (PF == 3) wload(2, wcx, scx);
    if constexpr (FULL) {
        // this wave's staging landed (it was issued before the 5 PF weight
        // loads in flight); the barrier below makes every wave's visible
        __builtin_amdgcn_s_waitcnt(VMCNT0 | (5 * PF));
    } else {
        commit(0, 0);
    }
    const v16i czero = {};  // the accumulator operand: an inline 0, no registers
    const int nsh = h ? 0 : 4;  // this half's nibble to the high half of each byte
    __syncthreads();

    // register groups holding entries of the item (8 entries per group)
    auto run = [&](auto ngc) {
        constexpr int NG = decltype(ngc)::value;
        // chunk ch from set w (scales sc); chunk ch + PF loads into set wl
        auto step = [&](int ch, uint4 (&w)[4], const uint4 &sc, uint4 (&wl)[4], uint4 &sl) {
            const int q = ch & 1;
            if constexpr (!FULL) {
                stage(ch + 1);
                __builtin_amdgcn_sched_barrier(0);  // activations issued before the weights
            }
            wload(ch + PF, wl, sl);
            if (ch < nch) {  // uniform
                const uint8_t *tq = FULL ? smem + ch * FA + n * 256
                                         : tokl + (size_t)q * M * MF_TS + (size_t)n * MF_TS + 16 * h;
                const float *xq = FULL ? reinterpret_cast<const float *>(smem + MS_FC * FA) + ch * FD + 4 * h
                                       : dxl + q * MF_KC * M + 4 * h;
                const uint32_t scw[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
                for (int bl = 0; bl < MF_KC; bl++) {
                    const int b = ch * MF_KC + bl;
                    // SCV: nb % MF_KC == 0, so every block of a chunk below nch
                    // exists; without the test the chunk is one basic block and
                    // the scheduler overlaps one block's epilogue with the next
                    // block's swaps and MFMA (the guard cost 16 register moves
                    // per chunk and 2-3 us of gate/up)
                    if (SCV || b < nb) {
                        // block bl sits in w[bl % 4] of the half bl / 4 lane: the swap
                        // at bl < 4 yields block bl and keeps block bl + 4 in w[bl]
                        uint4 blk;
                        if (bl < 4) {
                            uint4 &wr = w[bl];
                            half_split(wr.x, blk.x, wr.x);
                            half_split(wr.y, blk.y, wr.y);
                            half_split(wr.z, blk.z, wr.z);
                            half_split(wr.w, blk.w, wr.w);
                        } else {
                            blk = w[bl & 3];
                        }
                        // 16 (q - 8) per byte: ((q << 4) & 0xF0) ^ 0x80, exact in int8
                        v4i wq;
                        wq.x = (int)(((blk.x << nsh) & 0xF0F0F0F0u) ^ 0x80808080u);
                        wq.y = (int)(((blk.y << nsh) & 0xF0F0F0F0u) ^ 0x80808080u);
                        wq.z = (int)(((blk.z << nsh) & 0xF0F0F0F0u) ^ 0x80808080u);
                        wq.w = (int)(((blk.w << nsh) & 0xF0F0F0F0u) ^ 0x80808080u);
                        const v4i ta = FULL ? *reinterpret_cast<const v4i *>(tq + (((2 * bl + h + n) & 15) << 4))
                                            : *reinterpret_cast<const v4i *>(tq + bl * 32);
                        // (FULL: the staged scales are dx itself, so the 1/16 goes with dw;
                        // both are exact: powers of two)
                        const float dw = FULL ? h2f((uint16_t)(scw[bl >> 1] >> (16 * (bl & 1)))) * 0.0625f
                                              : h2f((uint16_t)(scw[bl >> 1] >> (16 * (bl & 1))));
                        float4 dx[NG];
#pragma unroll
                        for (int g = 0; g < NG; g++) dx[g] = *reinterpret_cast<const float4 *>(xq + bl * M + 8 * g);
                        // rc = 16 S exactly (|16 S| < 2^24): u16 = round(16 S * dw) =
                        // 16 round(S * dw), and u16 * (dx / 16) = round(S * dw) * dx
                        const v16i rc = __builtin_amdgcn_mfma_i32_32x32x32_i8(ta, wq, czero, 0, 0, 0);
#pragma unroll
                        for (int g = 0; g < NG; g++) {
                            const float dxa[4] = {dx[g].x, dx[g].y, dx[g].z, dx[g].w};
#pragma unroll
                            for (int rr = 0; rr < 4; rr++) {
                                const int r = 4 * g + rr;
                                const float u16 = (float)rc[r] * dw;
                                acc[r] = __builtin_fmaf(u16, dxa[rr], acc[r]);
                            }
                        }
                    }
                }
            }
            // unconditional (zeros past the last chunk), so the activation
            // loads stay ahead of the weight loads
            if constexpr (!FULL) {
                commit(q ^ 1, ch + 1);
                __syncthreads();
            }
        };
        if constexpr (PF == 3) {
            for (int ch = 0; ch < nch; ch += 4) {
                step(ch, wa, sa, wdx, sdx);
                step(ch + 1, wb, sbv, wa, sa);
                step(ch + 2, wcx, scx, wb, sbv);
                step(ch + 3, wdx, sdx, wcx, scx);
            }
        } else {
            for (int ch = 0; ch < nch; ch += 3) {
                step(ch, wa, sa, wcx, scx);
                step(ch + 1, wb, sbv, wa, sa);
                step(ch + 2, wcx, scx, wb, sbv);
            }
        }
    };
    const int ng = (c + 7) >> 3;
    if (ng >= 4) run(Tiles<4>{});
    else if (ng == 3) run(Tiles<3>{});
    else if (ng == 2) run(Tiles<2>{});
    else run(Tiles<1>{});

    if (PAIR) {
        // the pair's sums meet in LDS (over the activation buffers) and each
        // wave applies SwiGLU and Q8_0 to half of the entries: registers
        // r % 4 < 2 the gate wave, the others the up wave; each hands over
        // its sums of the other half.  Register groups past the item's
        // entries are skipped (uniform).
        float *x = reinterpret_cast<float *>(smem) + (size_t)(wave >> 1) * 16 * 64;
        if constexpr (FULL) __syncthreads();  // every wave is done with the staged activations
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const bool give = r < 4 * ng && (mat == 0) == ((r & 2) != 0);  // uniform
            if (give) x[r * 64 + lane] = acc[r];
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < 16; r++) {
            if (r >= 4 * ng) break;
            if ((mat == 0) == ((r & 2) != 0)) continue;  // the other wave's entry
            const int t = 8 * (r >> 2) + 4 * h + (r & 3);
            const bool on = valid && t < c;
            const float own = acc[r], other = x[r * 64 + lane];
            const float hv = on ? silu_mul(mat == 0 ? own : other, mat == 0 ? other : own) : 0.0f;
            const float v = fabsf(hv);
            const float a = half_max(v > 0.0f ? v : 0.0f);
            const float d = a / 127.0f;
            const float inv = a > 0.0f ? 127.0f / a : 0.0f;
            const int qv = (int)__builtin_rintf(hv * inv);
            const int sum = half_sum(qv);
            if (on) {
                const int ent = entries[o + t];
                int8_t *qp = oq + (size_t)ent * s.I + nt * 32 + n;
                const size_t si = (size_t)ent * s.nbI + nt;
                if constexpr (GD) {  // read by down blocks of this launch
                    __hip_atomic_store(qp, (int8_t)qv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (n == 0) {
                        st_coh(od + si, h2f(f2h(d)));
                        __hip_atomic_store(os + si, sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                } else {
                    *qp = (int8_t)qv;
                    if (n == 0) {
                        od[si] = h2f(f2h(d));
                        os[si] = sum;
                    }
                }
            }
        }
        if constexpr (GD) {
            __builtin_amdgcn_s_waitcnt(VMCNT0);  // this thread's h stores acknowledged
            __syncthreads();                     // ... every thread's
            if (tid == 0 && wi != G.drop)
                __hip_atomic_fetch_add(G.rdy + wi, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else {
        if (valid) {
            const bool coh = F.cnt != nullptr;  // uniform
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int t = 8 * (r >> 2) + 4 * h + (r & 3);
                if (t < c) {
                    float *dst = D + (size_t)entries[o + t] * s.H + nt * 32 + n;
                    const float v = gd_bad ? __builtin_nanf("") : acc[r];
                    if (coh)
                        st_coh(dst, v);
                    else
                        *dst = v;
                }
            }
        }
        // NW * 32 == FC_ROWS: block x covers output tile x
        if (F.cnt) fused_combine<NT>(F, s, entries, o, c, bx, D, smem);
    }
}

template <bool PAIR, bool SCV, bool FULL>
__global__ __launch_bounds__(MS_NW * 64) void k_mfma_small(const uint8_t *__restrict__ layer_pl, Shape s,
                                                           const int32_t *__restrict__ work,
                                                           const int32_t *__restrict__ work_n,
                                                           const int32_t *__restrict__ entries,
                                                           const int8_t *__restrict__ aq, const float *__restrict__ ad,
                                                           int8_t *__restrict__ oq, float *__restrict__ od,
                                                           int *__restrict__ os, float *__restrict__ D, FuseArgs F) {
    ms_item<PAIR, SCV, FULL, false>(layer_pl, s, work, work_n, entries, aq, ad, oq, od, os, D, F, (int)blockIdx.y,
                                    (int)blockIdx.x, GdArgs());
}

// Gate/up and down of the one-tile items in one launch: blocks [0, gxg wmax)
// are the gate/up blocks (item b / gxg, row tile b % gxg), the rest the down
// blocks.  Blocks are dispatched in order of their id on each XCD, so every
// gate/up block has been dispatched (and runs without waiting) before a down
// block of the same XCD takes a slot; a down block's wait ends once the
// gate/up blocks of its item, on whichever XCD, have stored h.  The down
// blocks then fill the slots the gate/up launch's last round leaves idle.
template <bool SCVG, bool FULLG>
__global__ __launch_bounds__(MS_NW * 64) void k_mfma_small_gd(const uint8_t *__restrict__ layer_pl, Shape s,
                                                              const int32_t *__restrict__ work,
                                                              const int32_t *__restrict__ work_n,
                                                              const int32_t *__restrict__ entries,
                                                              const int8_t *__restrict__ xq,
                                                              const float *__restrict__ xd, int8_t *hq, float *hd,
                                                              int *hs, float *__restrict__ D, GdArgs G, int gxg,
                                                              int gxd, int wmax) {
    const int b = (int)blockIdx.x, ng = gxg * wmax;
    if (b < ng) {
        ms_item<true, SCVG, FULLG, true>(layer_pl, s, work, work_n, entries, xq, xd, hq, hd, hs, nullptr, FuseArgs(),
                                         b / gxg, b % gxg, G);
    } else {
        const int d = b - ng;
        ms_item<false, true, true, true>(layer_pl, s, work, work_n, entries, hq, hd, nullptr, nullptr, nullptr, D,
                                         FuseArgs(), d / gxd, d % gxd, G);
    }
}

// ================================================================ 16 x 16 tiles
// The prefill / large-batch path.  Work item = (expert e, up to XT_CT * 16
// entries).  A block of NW waves stages, per chunk of XT_KC Q4_0 blocks, the
// item's activations and activation scales and every wave's weight rows and
// their scales straight into LDS (global_load_lds, no registers on the way;
// one wait and one barrier per chunk, the next chunk in flight meanwhile).
// Each wave owns 32 weight rows (two 16-row tiles) across the item's entries
// (16-entry column tiles) and runs one v_mfma_i32_16x16x32_i8 per (row
// tile, column tile, block): K = 32 is one Q4_0 / Q8_0 block.
//
// Operands (lane l, g = l / 16, c = l % 16; measured on gfx950):
//   A  row c of the row tile, block elements 8g .. 8g+7: the low (g < 2) or
//      high (g >= 2) nibbles of bytes 8 (g & 1) .. 8 (g & 1) + 7 of the row's
//      16, as 16 (q - 8) = ((q << 4) ^ 0x80) per byte (exact in int8)
//   B  entry c of the column tile, block elements 8g .. 8g+7 (Q8_0 bytes)
//   C  0x4B400000 for every element
// so D = 0x4B400000 + 16 S, |16 S| <= 520192 < 2^22: D's bits are the float
// 1.5 * 2^23 + 16 S exactly.  D's register r of lane l is (row 4g + r,
// entry c) of the tile.
// Epilogue per block, the row-dot definition bit for bit:
//   u   = fma(float_bits(D), dw / 16, -1.5 * 2^23 * dw / 16) = round(S * dw)
//         (dw / 16 and the constant are exact: dw is a half)
//   acc = fma(u, dx, acc)
// Each lane needs 4 row scales per row tile (its rows 4g .. 4g+3) and one
// activation scale per column tile (entry c).  Gate/up: waves 2i / 2i + 1
// take gate / up of the same 32 rows; the two hand each other half of their
// sums in LDS and each applies SwiGLU and Q8_0 to half of the column tiles
// (an entry's 32 rows sit in lanes c, c + 16, c + 32, c + 48, 8 values
// each).  Down writes fp32 rows.
constexpr int XT_NW = 4;     // waves per block
constexpr int XT_KC = 4;     // Q4_0 blocks per chunk
constexpr int XT_CT = 10;    // 16-entry column tiles per item (160 entries)
constexpr int XT_RB = XT_KC * 32;   // activation bytes per row and chunk
constexpr int XT_NP = XT_KC * 2;    // 16-byte pieces per row and chunk
constexpr int XT_CS = 12;           // activation-scale row: the column tiles' scales, then unused words (12
                                    // words apart, 16 consecutive rows' 16-byte reads fall on distinct banks)
static_assert(XT_CS >= XT_CT && XT_CS % 4 == 0, "scale row");

// LDS byte offsets of one block's buffers (two of each staged buffer)
struct XtLds {
    static constexpr int ROWS = XT_CT * 16;
    static constexpr int ACT = 0;                                     // [2][ROWS][XT_RB], pieces swizzled
    static constexpr int AXS = ACT + 2 * ROWS * XT_RB;                // [2][XT_KC][16][XT_CS] fp32
    static constexpr int WQ = AXS + 2 * XT_KC * 16 * XT_CS * 4;       // [3][NW][32 rows][XT_KC][16 B]
    static constexpr int WSR = WQ + 3 * XT_NW * 32 * XT_KC * 16;      // [3][NW][32 rows][XT_KC] halves
    static constexpr int TAB = WSR + 3 * XT_NW * 32 * XT_KC * 2;      // [NW][XT_KC][2][2 rt][16] fp32
    static constexpr int BYTES = TAB + XT_NW * XT_KC * 2 * 2 * 16 * 4;
};
static_assert(XtLds::ACT % 16 == 0 && XtLds::AXS % 16 == 0 && XtLds::WQ % 16 == 0 && XtLds::WSR % 16 == 0 &&
              XtLds::TAB % 16 == 0, "LDS alignment");
static_assert(XT_NP == 8, "piece swizzle assumes 8 pieces per row");
static_assert((XT_NW / 2) * 64 * (2 * XT_CT * 4) * 4 <= XtLds::BYTES, "gate/up hand-off fits in the block's LDS");

// 16-byte piece slot of piece p in activation row t (rows t and t + 2 fall
// on the same banks; the slot spreads 16 consecutive rows over all 64)
TG_DEV int xt_slot(int p, int t) { return p ^ ((t >> 1) & 7); }
// 16-byte block slot of block bl in weight row r of a wave
TG_DEV int xt_wslot(int bl, int r) { return bl ^ ((r >> 2) & 3); }

// 16 (q - 8) as int8 from 8 nibble bytes: low nibbles (sh = 4) or high (sh = 0)
TG_DEV long xt_unpack(uint2 w, int sh) {
    const uint32_t lo = ((w.x << sh) & 0xF0F0F0F0u) ^ 0x80808080u;
    const uint32_t hi = ((w.y << sh) & 0xF0F0F0F0u) ^ 0x80808080u;
    return (long)(((uint64_t)hi << 32) | lo);
}

// One block of the 16 x 16 kernels: item wi, row tile bx.  GD: gate/up and
// down blocks of the same launch (k_mfma16_gd), as in the one-tile kernels:
// a gate/up block stores h at agent scope and counts itself in at rdy[wi]
// once the stores are acknowledged; a down block waits (bounded) for all
// `need` gate/up blocks of its item and stages h at agent scope.
template <bool PAIR, bool GD>
TG_DEV __attribute__((always_inline)) void x16_item(const uint8_t *__restrict__ layer_pl, const Shape s,
                                                    const int32_t *__restrict__ work,
                                                    const int32_t *__restrict__ work_n,
                                                    const int32_t *__restrict__ entries,
                                                    const int8_t *__restrict__ aq, const float *__restrict__ ad,
                                                    int8_t *__restrict__ oq, float *__restrict__ od,
                                                    int *__restrict__ os, float *__restrict__ D, const FuseArgs F,
                                                    int wi, int bx, const GdArgs G) {
    // the launch's dynamic LDS, named here so its addresses stay LDS
    // addresses (through a generic pointer each cast to LDS adds a null test)
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int NW = XT_NW, ROWS = XtLds::ROWS;
    constexpr int NACT = ROWS * XT_NP / 64;          // activation load instructions per chunk (full item)
    constexpr int NAXS = XT_KC * 16 * XT_CS / 64;    // activation-scale load instructions per chunk
    static_assert(NACT % NW == 0 && NAXS % NW == 0, "staging split");
    if (wi >= work_n[0]) return;  // uniform over the block
    const int e = work[3 * wi], o = work[3 * wi + 1], c = work[3 * wi + 2];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, cl = lane & 15;
    const int K = PAIR ? s.H : s.I, nb = K / QK, k = s.k;
    const int nch = nb / XT_KC;
    const int ct_n = (c + 15) >> 4;                  // column tiles holding entries

    // activation row (token for gate/up, entry for down) of item entry t;
    // rows past the item's last entry read its first row (never stored)
    auto arow = [&](int t) -> int {
        const int ent = entries[o + (t < c ? t : 0)];
        return PAIR ? ent / k : ent;
    };
    // staging maps, fixed over the chunks: activation piece and scale sources
    int aoff[NACT / NW], soff[NAXS / NW];
#pragma unroll
    for (int u = 0; u < NACT / NW; u++) {
        const int j = u * NW + wave, i = j * 64 + lane, t = i / XT_NP, sl = i % XT_NP;
        aoff[u] = arow(t) * K + xt_slot(sl, t) * 16;  // ^ is an involution: slot sl holds piece xt_slot(sl, t)
    }
#pragma unroll
    for (int u = 0; u < NAXS / NW; u++) {
        const int j = u * NW + wave, d = j * 64 + lane, bl = d / (16 * XT_CS), rem = d % (16 * XT_CS);
        const int cs = rem % XT_CS, t = (cs < XT_CT ? cs : 0) * 16 + rem / XT_CS;  // padding words: any row
        soff[u] = arow(t) * nb + bl;
    }
    // this wave's 32 weight rows
    const int mat = PAIR ? (wave & 1) : 0;  // 0 gate / down, 1 up
    const int rb = PAIR ? (bx * (NW / 2) + (wave >> 1)) * 32 : (bx * NW + wave) * 32;
    const uint8_t *ex = layer_pl + (size_t)e * s.EB;
    const uint8_t *tb = PAIR ? ex + (size_t)mat * s.GB : ex + 2 * s.GB;
    const int rows = PAIR ? s.I : s.H;
    const uint8_t *wrow = tb + (size_t)rb * nb * 16;
    const uint8_t *wsc = tb + (size_t)rows * nb * 16 + (size_t)rb * nb * 2;
    // weight staging: lane l -> row l / 4 (+16), slot l % 4; scales: row l / 2, half-pair l % 2
    const int wr0 = lane >> 2, wsl = lane & 3;
    const int woff0 = wr0 * nb * 16 + xt_wslot(wsl, wr0) * 16;
    const int woff1 = (wr0 + 16) * nb * 16 + xt_wslot(wsl, wr0 + 16) * 16;
    const int soffw = (lane >> 1) * nb * 2 + (lane & 1) * 4;

    // activations and their scales: one chunk ahead, two buffers (GD down
    // blocks: h of this launch, at agent scope)
    constexpr bool COH = GD && !PAIR;
    auto stage_act = [&](int ch) {
        const int q = ch & 1;
#pragma unroll
        for (int u = 0; u < NACT / NW; u++) {
            const int j = u * NW + wave;
            if (j * 64 < ct_n * 16 * XT_NP) {  // rows of column tiles in use (uniform per instruction)
                const uint32_t m0 = lds_addr(smem, XtLds::ACT + q * ROWS * XT_RB + j * 1024);
                if constexpr (COH)
                    lds_dma16_coh(aq + aoff[u] + ch * XT_RB, m0);
                else
                    lds_dma16(aq + aoff[u] + ch * XT_RB, m0);
            }
        }
#pragma unroll
        for (int u = 0; u < NAXS / NW; u++) {
            const int j = u * NW + wave;
            const uint32_t m0 = lds_addr(smem, XtLds::AXS + (q * XT_KC * 16 * XT_CS + j * 64) * 4);
            if constexpr (COH)
                lds_dma4_coh(ad + soff[u] + ch * XT_KC, m0);
            else
                lds_dma4(ad + soff[u] + ch * XT_KC, m0);
        }
    };
    // the wave's weight rows and their scales (streamed from HBM): two
    // chunks ahead, three buffers; XT_WLOADS load instructions per thread
    constexpr int XT_WLOADS = 3;
    auto stage_w = [&](int ch) {
        const int q = ch % 3;
        const int wq = XtLds::WQ + (q * NW + wave) * 32 * XT_KC * 16;
        lds_dma16(wrow + woff0 + ch * XT_KC * 16, lds_addr(smem, wq));
        lds_dma16(wrow + woff1 + ch * XT_KC * 16, lds_addr(smem, wq + 1024));
        lds_dma4(wsc + soffw + ch * XT_KC * 2, lds_addr(smem, XtLds::WSR + (q * NW + wave) * 32 * XT_KC * 2));
    };

    float acc[2][XT_CT][4];
#pragma unroll
    for (int rt = 0; rt < 2; rt++)
#pragma unroll
        for (int ct = 0; ct < XT_CT; ct++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[rt][ct][r] = 0.0f;
    v4i cmag;
#pragma unroll
    for (int r = 0; r < 4; r++) cmag[r] = (int)MAGIC_I;

    float *tab = reinterpret_cast<float *>(smem + XtLds::TAB) + wave * XT_KC * 2 * 2 * 16;
    const int sh = g < 2 ? 4 : 0;  // low nibbles for elements 0..15, high for 16..31

    // GD down block: every gate/up block of the item has counted in
    // (bounded; when the wait runs out the rows are stored as NaN and *err
    // set).  Its first weight chunk is in flight meanwhile.
    bool gd_bad = false;
    if constexpr (COH) {
        __shared__ int gd_flag;
        stage_w(0);
        if (tid == 0) {
            uint32_t tries = 0;
            int bad = 0;
            while (__hip_atomic_load(G.rdy + wi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < G.need) {
                if (++tries >= G.spin) {
                    bad = 1;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            gd_flag = bad;
            if (bad) __hip_atomic_store(G.err, 4u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        gd_bad = gd_flag != 0;
        stage_act(0);
        if (nch > 1) stage_w(1);
    } else {
        // issue order: w(0), act(0), w(1); then per chunk ch: act(ch + 1), w(ch + 2)
        stage_w(0);
        stage_act(0);
        if (nch > 1) stage_w(1);
    }
    auto run = [&](auto ctv) {
        constexpr int CT = decltype(ctv)::value;
        for (int ch = 0; ch < nch; ch++) {
            const int q = ch & 1, qw = ch % 3;
            // this thread's loads of chunk ch are in LDS: everything but w(ch + 1), issued last, if issued
            if (ch + 1 < nch)
                __builtin_amdgcn_s_waitcnt(VMCNT0 | XT_WLOADS);
            else
                __builtin_amdgcn_s_waitcnt(VMCNT0);
            __syncthreads();  // everyone's; and chunk ch - 1 is read by all
            if (ch + 1 < nch) stage_act(ch + 1);
            if (ch + 2 < nch) stage_w(ch + 2);
            // row scales of the chunk: dw / 16 and -1.5 * 2^23 * dw / 16, by lanes 0..31 (row = lane)
            if (lane < 32) {
                const uint2 hv = *reinterpret_cast<const uint2 *>(smem + XtLds::WSR +
                                                                  ((qw * NW + wave) * 32 + lane) * XT_KC * 2);
                const uint16_t hs[4] = {(uint16_t)hv.x, (uint16_t)(hv.x >> 16), (uint16_t)hv.y,
                                        (uint16_t)(hv.y >> 16)};
#pragma unroll
                for (int bl = 0; bl < XT_KC; bl++) {
                    const float d16 = h2f(hs[bl]) * 0.0625f;
                    float *tt = tab + bl * 64 + (lane >> 4) * 16 + (lane & 15);
                    tt[0] = d16;
                    tt[32] = -MAGIC_F * d16;
                }
            }
            wave_lds_sync();
            const uint8_t *act = smem + XtLds::ACT + q * ROWS * XT_RB;
            const float *axs = reinterpret_cast<const float *>(smem + XtLds::AXS) + q * XT_KC * 16 * XT_CS;
            const uint8_t *wq = smem + XtLds::WQ + (qw * NW + wave) * 32 * XT_KC * 16;
            // one block's operands: raw weight bytes (unpacked on use), row scales, activation scales and bytes
            struct Ops {
                uint2 w[2];
                float dw[2][4], cw[2][4];
                float dx[XT_CS];
                long b[CT];
            };
            auto load = [&](int bl, Ops &o) {
#pragma unroll
                for (int rt = 0; rt < 2; rt++) {
                    const int r = rt * 16 + cl;
                    o.w[rt] = *reinterpret_cast<const uint2 *>(wq + r * XT_KC * 16 + xt_wslot(bl, r) * 16 + 8 * (g & 1));
                    const float4 v = *reinterpret_cast<const float4 *>(tab + bl * 64 + rt * 16 + 4 * g);
                    const float4 u = *reinterpret_cast<const float4 *>(tab + bl * 64 + 32 + rt * 16 + 4 * g);
                    o.dw[rt][0] = v.x; o.dw[rt][1] = v.y; o.dw[rt][2] = v.z; o.dw[rt][3] = v.w;
                    o.cw[rt][0] = u.x; o.cw[rt][1] = u.y; o.cw[rt][2] = u.z; o.cw[rt][3] = u.w;
                }
#pragma unroll
                for (int c4 = 0; c4 < (CT + 3) / 4; c4++) {
                    const float4 v = *reinterpret_cast<const float4 *>(axs + (bl * 16 + cl) * XT_CS + 4 * c4);
                    o.dx[4 * c4] = v.x; o.dx[4 * c4 + 1] = v.y; o.dx[4 * c4 + 2] = v.z; o.dx[4 * c4 + 3] = v.w;
                }
                const int p = bl * 2 + (g >> 1);
#pragma unroll
                for (int ct = 0; ct < CT; ct++) {
                    const int t = ct * 16 + cl;
                    o.b[ct] = *reinterpret_cast<const long *>(act + t * XT_RB + xt_slot(p, t) * 16 + 8 * (g & 1));
                }
            };
            // block products: product i = (column tile i / 2, row tile i % 2);
            // product i + 1 is issued before product i's epilogue (two result
            // sets), and the next block's product 0 before this block's last
            // epilogue (the last product is odd: it uses set 1, product 0 set 0)
            v4i dq0, dq1;
            long a[2];
            auto compute = [&](const Ops &o, const Ops &nx, auto has_next) {
                constexpr bool HN = decltype(has_next)::value != 0;
                long an[2] = {0, 0};
#pragma unroll
                for (int i = 0; i < 2 * CT; i++) {
                    const int ct = i >> 1, rt = i & 1;
                    __builtin_amdgcn_sched_barrier(0);
                    if (i + 1 < 2 * CT) {
                        const v4i m = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[(i + 1) & 1], o.b[(i + 1) >> 1], cmag,
                                                                            0, 0, 0);
                        if (i & 1) dq0 = m; else dq1 = m;
                    } else if constexpr (HN) {
                        an[0] = xt_unpack(nx.w[0], sh);
                        an[1] = xt_unpack(nx.w[1], sh);
                        dq0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(an[0], nx.b[0], cmag, 0, 0, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    const v4i d = (i & 1) ? dq1 : dq0;
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float u = __builtin_fmaf(__int_as_float(d[r]), o.dw[rt][r], o.cw[rt][r]);
                        acc[rt][ct][r] = __builtin_fmaf(u, o.dx[ct], acc[rt][ct][r]);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                a[0] = an[0];
                a[1] = an[1];
            };
            // two operand sets in turn: block bl + 1's loads are in flight during block bl's products
            static_assert(XT_KC % 2 == 0, "blocks per chunk in pairs");
            Ops oa, ob;
            load(0, oa);
            a[0] = xt_unpack(oa.w[0], sh);
            a[1] = xt_unpack(oa.w[1], sh);
            dq0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[0], oa.b[0], cmag, 0, 0, 0);
#pragma unroll
            for (int bl = 0; bl < XT_KC; bl += 2) {
                load(bl + 1, ob);
                compute(oa, ob, Tiles<1>{});
                if (bl + 2 < XT_KC) {
                    load(bl + 2, oa);
                    compute(ob, oa, Tiles<1>{});
                } else {
                    compute(ob, oa, Tiles<0>{});
                }
            }
        }
    };
    // the item's column tiles (below 6 rounded up to an even count)
    if (ct_n > 9) run(Tiles<10>{});
    else if (ct_n > 8) run(Tiles<9>{});
    else if (ct_n > 7) run(Tiles<8>{});
    else if (ct_n > 6) run(Tiles<7>{});
    else if (ct_n > 4) run(Tiles<6>{});
    else if (ct_n > 2) run(Tiles<4>{});
    else run(Tiles<2>{});
    __syncthreads();  // the staging buffers are free for the hand-off

    if (PAIR) {
        // the pair's sums meet in LDS and each wave applies SwiGLU and Q8_0
        // to half of the item's column tiles, the gate wave to [0, hc) and the
        // up wave to [hc, ct_n): each hands over its sums of the other half
        // (the LDS slots of one whole hand-over)
        float *x = reinterpret_cast<float *>(smem) + (size_t)(wave >> 1) * 64 * 2 * XT_CT * 4;
        const int hc = (ct_n + 1) >> 1;
#pragma unroll
        for (int ct = 0; ct < XT_CT; ct++) {
            const bool give = mat == 0 ? (ct >= hc && ct < ct_n) : ct < hc;  // uniform
            if (give) {
#pragma unroll
                for (int rt = 0; rt < 2; rt++)
#pragma unroll
                    for (int r = 0; r < 4; r++) x[((rt * XT_CT + ct) * 4 + r) * 64 + lane] = acc[rt][ct][r];
            }
        }
        __syncthreads();
        const int nt = rb >> 5;  // I-block of the 32 rows
#pragma unroll
        for (int ct = 0; ct < XT_CT; ct++) {
            const bool mine = mat == 0 ? ct < hc : (ct >= hc && ct < ct_n);  // uniform
            if (!mine) continue;
            const int t = ct * 16 + cl;
            const bool on = t < c;
            float hv[2][4], a = 0.0f;
#pragma unroll
            for (int rt = 0; rt < 2; rt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float own = acc[rt][ct][r], other = x[((rt * XT_CT + ct) * 4 + r) * 64 + lane];
                    hv[rt][r] = on ? silu_mul(mat == 0 ? own : other, mat == 0 ? other : own) : 0.0f;
                    const float v = fabsf(hv[rt][r]);
                    a = v > a ? v : a;
                }
            float ao = __shfl_xor(a, 16, WAVE);
            a = ao > a ? ao : a;
            ao = __shfl_xor(a, 32, WAVE);
            a = ao > a ? ao : a;
            const float d = a / 127.0f;
            const float inv = a > 0.0f ? 127.0f / a : 0.0f;
            int qv[2][4], sum = 0;
#pragma unroll
            for (int rt = 0; rt < 2; rt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    qv[rt][r] = (int)__builtin_rintf(hv[rt][r] * inv);
                    sum += qv[rt][r];
                }
            sum += __shfl_xor(sum, 16, WAVE);
            sum += __shfl_xor(sum, 32, WAVE);
            if (on) {
                const int ent = entries[o + t];
                int8_t *dst = oq + (size_t)ent * s.I + rb + 4 * g;
                const size_t si = (size_t)ent * s.nbI + nt;
#pragma unroll
                for (int rt = 0; rt < 2; rt++) {
                    const uint32_t w = (uint32_t)(qv[rt][0] & 0xFF) | ((uint32_t)(qv[rt][1] & 0xFF) << 8) |
                                       ((uint32_t)(qv[rt][2] & 0xFF) << 16) | ((uint32_t)(qv[rt][3] & 0xFF) << 24);
                    uint32_t *wp = reinterpret_cast<uint32_t *>(dst + 16 * rt);
                    if constexpr (GD)  // read by down blocks of this launch
                        __hip_atomic_store(wp, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    else
                        *wp = w;
                }
                if (g == 0) {
                    if constexpr (GD) {
                        st_coh(od + si, h2f(f2h(d)));
                        __hip_atomic_store(os + si, sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    } else {
                        od[si] = h2f(f2h(d));
                        os[si] = sum;
                    }
                }
            }
        }
        if constexpr (GD) {
            __builtin_amdgcn_s_waitcnt(VMCNT0);  // this thread's h stores acknowledged
            __syncthreads();                     // ... every thread's
            if (tid == 0 && wi != G.drop)
                __hip_atomic_fetch_add(G.rdy + wi, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else {
        const bool coh = F.cnt != nullptr;  // uniform
#pragma unroll
        for (int ct = 0; ct < XT_CT; ct++) {
            const int t = ct * 16 + cl;
            if (t < c) {
                float *dst = D + (size_t)entries[o + t] * s.H + rb + 4 * g;
#pragma unroll
                for (int rt = 0; rt < 2; rt++) {
                    float v[4];
#pragma unroll
                    for (int r = 0; r < 4; r++) v[r] = gd_bad ? __builtin_nanf("") : acc[rt][ct][r];
                    if (coh) {
                        st_coh2(dst + 16 * rt, v[0], v[1]);
                        st_coh2(dst + 16 * rt + 2, v[2], v[3]);
                    } else {
                        *reinterpret_cast<float4 *>(dst + 16 * rt) = make_float4(v[0], v[1], v[2], v[3]);
                    }
                }
            }
        }
        // NW * 32 == FC_ROWS: the block's rows are output tile bx
        if (F.cnt) fused_combine<XT_NW * 64>(F, s, entries, o, c, bx, D, smem);
    }
}

// blocks are dealt to the 8 XCDs in turn (block b on XCD b % 8): the gx
// blocks of one item get ids 8 apart, so they share one XCD's L2 (the
// item's activations are fetched into one L2, not eight)
TG_DEV void x16_place(int bid, int gx, int &wi, int &bx) {
    const int rest = bid >> 3;
    bx = rest % gx;
    wi = (rest / gx) * 8 + (bid & 7);
}

template <bool PAIR>
__global__ __launch_bounds__(XT_NW * 64) void k_mfma16(const uint8_t *__restrict__ layer_pl, Shape s,
                                                       const int32_t *__restrict__ work,
                                                       const int32_t *__restrict__ work_n,
                                                       const int32_t *__restrict__ entries,
                                                       const int8_t *__restrict__ aq, const float *__restrict__ ad,
                                                       int8_t *__restrict__ oq, float *__restrict__ od,
                                                       int *__restrict__ os, float *__restrict__ D, FuseArgs F) {
    const int gx = PAIR ? s.I / (32 * (XT_NW / 2)) : s.H / (32 * XT_NW);
    int wi, bx;
    x16_place((int)blockIdx.x, gx, wi, bx);
    x16_item<PAIR, false>(layer_pl, s, work, work_n, entries, aq, ad, oq, od, os, D, F, wi, bx, GdArgs());
}

// Gate/up and down of the 16 x 16 items in one launch: blocks [0, gxg wm8)
// are the gate/up blocks, the rest the down blocks (each part placed as in
// k_mfma16).  Blocks are dispatched in id order on each XCD and gate/up
// blocks never wait, so the down blocks' waits end (as in k_mfma_small_gd);
// the down blocks of the items done first fill the gate/up launch's tail.
__global__ __launch_bounds__(XT_NW * 64) void k_mfma16_gd(const uint8_t *__restrict__ layer_pl, Shape s,
                                                          const int32_t *__restrict__ work,
                                                          const int32_t *__restrict__ work_n,
                                                          const int32_t *__restrict__ entries,
                                                          const int8_t *__restrict__ xq, const float *__restrict__ xd,
                                                          int8_t *hq, float *hd, int *hs, float *__restrict__ D,
                                                          GdArgs G, int gxg, int gxd, int wm8) {
    const int b = (int)blockIdx.x, ng = gxg * wm8;
    int wi, bx;
    if (b < ng) {
        x16_place(b, gxg, wi, bx);
        x16_item<true, true>(layer_pl, s, work, work_n, entries, xq, xd, hq, hd, hs, nullptr, FuseArgs(), wi, bx, G);
    } else {
        x16_place(b - ng, gxd, wi, bx);
        x16_item<false, true>(layer_pl, s, work, work_n, entries, hq, hd, nullptr, nullptr, nullptr, D, FuseArgs(),
                              wi, bx, G);
    }
}

// ================================================================ launchers
static inline unsigned mf_cdiv(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }

// The dynamic-LDS limit of kernel fn raised to `bytes` (above 64 KB) on the
// current device, once per (kernel, device): `done` holds a bit per device.
static hipError_t lds_attr(const void *fn, size_t bytes, std::atomic<uint64_t> &done) {
    if (bytes <= 65536) return hipSuccess;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = dev >= 0 && dev < 64 ? 1ull << dev : 0;
    if (bit && (done.load(std::memory_order_relaxed) & bit)) return hipSuccess;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_relaxed);
    return e;
}

static bool x16_ok(const Shape &s, bool pair);

// entries per work item of the MFMA path at mt M-tiles: the 16 x 16 kernels
// take up to XT_CT * 16 (both of them must fit the shape)
// Shader clock under int8 MFMA load: every wave of the grid runs `iters`
// rounds of four independent v_mfma_i32_16x16x32_i8 chains and records
// s_memtime (shader clock cycles) and s_memrealtime (a 100 MHz counter)
// before and after them; lane 0 of each block's first wave stores the four
// stamps at out[4 * block].
__global__ __launch_bounds__(256) void k_clock_mfma(unsigned long long *out, int iters) {
    const int tid = threadIdx.x;
    __builtin_amdgcn_sched_barrier(0);
    const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    __builtin_amdgcn_sched_barrier(0);
    // operands depend on the stamp, so no MFMA can be placed before it
    const long a = (long)(0x0102030405060708ull ^ (t0 >> 62)) + tid, b = (long)0x0807060504030201ll - tid;
    v4i c0 = {0, 0, 0, 0}, c1 = c0, c2 = c0, c3 = c0;
    for (int i = 0; i < iters; i++) {
        c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(b, a, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, a, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_16x16x32_i8(b, b, c3, 0, 0, 0);
    }
    const int sink = c0.x + c1.y + c2.z + c3.w;
    __builtin_amdgcn_sched_barrier(0);
    const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    __builtin_amdgcn_sched_barrier(0);
    if (tid == 0) {
        unsigned long long *o = out + 4 * (size_t)blockIdx.x;
        o[0] = t0;
        o[1] = r0;
        o[2] = t1 + (sink == 0x7FFFFFFF ? 1u : 0u);  // keeps the chains
        o[3] = r1;
    }
}

hipError_t launch_clock_mfma(unsigned long long *out, int blocks, int iters, hipStream_t st) {
    TG_LAUNCH(k_clock_mfma, dim3(blocks), dim3(256), 0, st, out, iters);
    return hipGetLastError();
}

int mfma_item_entries(const Shape &s, int mt) {
    return mt == 4 && x16_ok(s, true) && x16_ok(s, false) ? XT_CT * 16 : 32 * mt;
}

int mfma_tiles(const Shape &s, int T) {
    // entries per expert in a work item: up to 4 M-tiles of 32; fewer when
    // the batch is small or the LDS staging would not fit
    const int avg = (T * s.k + s.E - 1) / s.E;
    return avg > 64 ? 4 : (avg > 16 ? 2 : 1);
}

bool mfma_shape_ok(const Shape &s) {
    return s.I % 32 == 0 && s.H % 32 == 0 && s.k <= MAX_K;
}

template <int MT, bool PAIR, int NW = mf_waves(MT)>
static hipError_t mf_go(const uint8_t *layer_pl, const Shape &s, int wmax, const int32_t *work, const int32_t *work_n,
                        const int32_t *entries, const int8_t *aq, const float *ad, int8_t *oq, float *od, int *os,
                        float *D, hipStream_t st) {
    const int rows = PAIR ? s.I : s.H;
    const size_t lds = mf_lds_bytes(MT, NW);
    const void *fn = reinterpret_cast<const void *>(&k_mfma_grouped<MT, PAIR, NW>);
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    // gate/up: NW/2 tiles (each as a gate wave and an up wave) per block
    const unsigned gx = PAIR ? mf_cdiv((size_t)rows, 32 * (NW / 2)) : mf_cdiv((size_t)rows, 32 * NW);
    TG_LAUNCH((k_mfma_grouped<MT, PAIR, NW>), dim3(gx, wmax), dim3(NW * 64), lds, st, layer_pl, s, work,
                       work_n, entries, aq, ad, oq, od, os, D);
    return hipGetLastError();
}

template <bool PAIR>
static hipError_t ms_go(const uint8_t *layer_pl, const Shape &s, int wmax, const int32_t *work, const int32_t *work_n,
                        const int32_t *entries, const int8_t *aq, const float *ad, int8_t *oq, float *od, int *os,
                        float *D, const FuseArgs &F, hipStream_t st) {
    static_assert(MS_NW * 32 == FC_ROWS && XT_NW * 32 == FC_ROWS, "one down block per output tile");
    const int rows = PAIR ? s.I : s.H, nb = (PAIR ? s.H : s.I) / QK;
    const unsigned gx = PAIR ? mf_cdiv((size_t)rows, 32 * (MS_NW / 2)) : mf_cdiv((size_t)rows, 32 * MS_NW);
    // whole chunks, at most MS_FC of them: the activations staged once (TG_MS_FULL=0: per chunk)
    static const bool full_on = [] {
        const char *v = getenv("TG_MS_FULL");
        return !(v && v[0] == '0');
    }();
    if (full_on && nb % MF_KC == 0 && nb <= MS_FC * MF_KC) {
        const size_t lds = ms_full_lds_bytes();
        static std::atomic<uint64_t> attr{0};
        hipError_t e = lds_attr(reinterpret_cast<const void *>(&k_mfma_small<PAIR, true, true>), lds, attr);
        if (e != hipSuccess) return e;
        TG_LAUNCH((k_mfma_small<PAIR, true, true>), dim3(gx, wmax), dim3(MS_NW * 64), lds, st, layer_pl, s, work,
                  work_n, entries, aq, ad, oq, od, os, D, F);
        return hipGetLastError();
    }
    const size_t lds = ms_lds_bytes();
    // 16-byte scale loads need every row's scales 16-byte aligned (nb % 8 == 0)
    if (nb % MF_KC == 0)
        TG_LAUNCH((k_mfma_small<PAIR, true, false>), dim3(gx, wmax), dim3(MS_NW * 64), lds, st, layer_pl, s, work,
                           work_n, entries, aq, ad, oq, od, os, D, F);
    else
        TG_LAUNCH((k_mfma_small<PAIR, false, false>), dim3(gx, wmax), dim3(MS_NW * 64), lds, st, layer_pl, s, work,
                           work_n, entries, aq, ad, oq, od, os, D, F);
    return hipGetLastError();
}

// the 16 x 16 kernel: whole chunks of K, whole 32-row groups per block
static bool x16_ok(const Shape &s, bool pair) {
    static const bool on = [] {
        const char *v = getenv("TG_MFMA16");
        return !(v && v[0] == '0');
    }();
    const int nb = (pair ? s.H : s.I) / QK, rows = pair ? s.I : s.H;
    return on && nb % XT_KC == 0 && rows % (pair ? 32 * (XT_NW / 2) : 32 * XT_NW) == 0;
}

template <bool PAIR>
static hipError_t x16_go(const uint8_t *layer_pl, const Shape &s, int wmax, const int32_t *work,
                         const int32_t *work_n, const int32_t *entries, const int8_t *aq, const float *ad, int8_t *oq,
                         float *od, int *os, float *D, const FuseArgs &F, hipStream_t st) {
    const unsigned gx = PAIR ? (unsigned)(s.I / (32 * (XT_NW / 2))) : (unsigned)(s.H / (32 * XT_NW));
    static std::atomic<uint64_t> attr{0};
    hipError_t e = lds_attr(reinterpret_cast<const void *>(&k_mfma16<PAIR>), XtLds::BYTES, attr);
    if (e != hipSuccess) return e;
    // one dimension: gx blocks for each of wmax items, wmax rounded up to 8
    const unsigned wm8 = (unsigned)((wmax + 7) / 8 * 8);
    TG_LAUNCH((k_mfma16<PAIR>), dim3(gx * wm8), dim3(XT_NW * 64), XtLds::BYTES, st, layer_pl, s, work, work_n,
              entries, aq, ad, oq, od, os, D, F);
    return hipGetLastError();
}

hipError_t launch_gateup_mfma(const uint8_t *layer_pl, const Shape &s, int mt, int wmax, const int32_t *work,
                              const int32_t *work_n, const int32_t *entries, const int8_t *xq, const float *xd,
                              const int *xs, int8_t *hq, float *hd, int *hs, hipStream_t st) {
    if (!mfma_shape_ok(s)) return hipErrorInvalidValue;
    (void)xs;
    const FuseArgs none;
    if (mt == 1) return ms_go<true>(layer_pl, s, wmax, work, work_n, entries, xq, xd, hq, hd, hs, nullptr, none, st);
    if (mt == 2) return mf_go<2, true>(layer_pl, s, wmax, work, work_n, entries, xq, xd, hq, hd, hs, nullptr, st);
    if (mfma_item_entries(s, mt) > 128)
        return x16_go<true>(layer_pl, s, wmax, work, work_n, entries, xq, xd, hq, hd, hs, nullptr, none, st);
    return mf_go<4, true>(layer_pl, s, wmax, work, work_n, entries, xq, xd, hq, hd, hs, nullptr, st);
}

// The kernels that can fold the combine in: the one-tile and the 16 x 16
// down kernels (blocks of FC_ROWS output rows).  Off unless TG_FUSE_COMBINE
// is 1 (read per call): the fold is bit-exact but measured slower than the
// separate k_combine launch, since each down block then waits for its
// stores, its arrival counts and its coherent loads in turn.
bool down_fuses(const Shape &s, int mt, int T) {
    const char *v = getenv("TG_FUSE_COMBINE");
    const bool on = v && v[0] == '1';
    const bool kern = mt == 1 || (mt == 4 && mfma_item_entries(s, mt) > 128);
    return on && kern && s.H % FC_ROWS == 0 && (size_t)T * s.k * s.H < ((size_t)1 << 31);
}

hipError_t launch_down_mfma(const uint8_t *layer_pl, const Shape &s, int mt, int wmax, const int32_t *work,
                            const int32_t *work_n, const int32_t *entries, const int8_t *hq, const float *hd,
                            const int *hs, float *D, const FuseArgs &F, hipStream_t st) {
    if (!mfma_shape_ok(s)) return hipErrorInvalidValue;
    (void)hs;
    if (mt == 1) return ms_go<false>(layer_pl, s, wmax, work, work_n, entries, hq, hd, nullptr, nullptr, nullptr,
                                     D, F, st);
    if (mt == 4 && mfma_item_entries(s, mt) > 128)
        return x16_go<false>(layer_pl, s, wmax, work, work_n, entries, hq, hd, nullptr, nullptr, nullptr, D, F,
                             st);
    if (F.cnt) return hipErrorInvalidValue;  // the kernels below leave the combine to k_combine
    if (mt == 2) return mf_go<2, false>(layer_pl, s, wmax, work, work_n, entries, hq, hd, nullptr, nullptr, nullptr,
                                        D, st);
    return mf_go<4, false>(layer_pl, s, wmax, work, work_n, entries, hq, hd, nullptr, nullptr, nullptr, D, st);
}

bool gd_fuses(const Shape &s, int mt) {
    const char *v = getenv("TG_FUSE_GD");
    const bool on = !(v && v[0] == '0');
    return on && mt == 1 && mfma_shape_ok(s) && s.nbI % MF_KC == 0 && s.nbI <= MS_FC * MF_KC;
}

bool gd16_fuses(const Shape &s, int mt) {
    const char *v = getenv("TG_FUSE_GD16");
    const bool on = !(v && v[0] == '0');
    return on && mt == 4 && mfma_shape_ok(s) && mfma_item_entries(s, mt) > 128 && x16_ok(s, true) &&
           x16_ok(s, false);
}

hipError_t launch_gu_down_x16(const uint8_t *layer_pl, const Shape &s, int wmax, const int32_t *work,
                              const int32_t *work_n, const int32_t *entries, const int8_t *xq, const float *xd,
                              int8_t *hq, float *hd, int *hs, float *D, const GdArgs &G0, hipStream_t st) {
    if (!gd16_fuses(s, 4) || !G0.rdy || !G0.err || G0.spin == 0) return hipErrorInvalidValue;
    const int gxg = s.I / (32 * (XT_NW / 2)), gxd = s.H / (32 * XT_NW), wm8 = (wmax + 7) / 8 * 8;
    if ((size_t)(gxg + gxd) * (size_t)wm8 >= ((size_t)1 << 31)) return hipErrorInvalidValue;
    GdArgs G = G0;
    G.need = gxg;
    static std::atomic<uint64_t> attr{0};
    hipError_t e = lds_attr(reinterpret_cast<const void *>(&k_mfma16_gd), XtLds::BYTES, attr);
    if (e != hipSuccess) return e;
    TG_LAUNCH(k_mfma16_gd, dim3((unsigned)((gxg + gxd) * wm8)), dim3(XT_NW * 64), XtLds::BYTES, st, layer_pl, s,
              work, work_n, entries, xq, xd, hq, hd, hs, D, G, gxg, gxd, wm8);
    return hipGetLastError();
}

template <bool SCVG, bool FULLG>
static hipError_t gd_go(const uint8_t *layer_pl, const Shape &s, int wmax, const int32_t *work,
                        const int32_t *work_n, const int32_t *entries, const int8_t *xq, const float *xd, int8_t *hq,
                        float *hd, int *hs, float *D, const GdArgs &G, int gxg, int gxd, hipStream_t st) {
    const size_t lds = ms_full_lds_bytes();
    static std::atomic<uint64_t> attr{0};
    hipError_t e = lds_attr(reinterpret_cast<const void *>(&k_mfma_small_gd<SCVG, FULLG>), lds, attr);
    if (e != hipSuccess) return e;
    TG_LAUNCH((k_mfma_small_gd<SCVG, FULLG>), dim3((unsigned)((gxg + gxd) * wmax)), dim3(MS_NW * 64), lds, st,
              layer_pl, s, work, work_n, entries, xq, xd, hq, hd, hs, D, G, gxg, gxd, wmax);
    return hipGetLastError();
}

hipError_t launch_gu_down_ms(const uint8_t *layer_pl, const Shape &s, int wmax, const int32_t *work,
                             const int32_t *work_n, const int32_t *entries, const int8_t *xq, const float *xd,
                             int8_t *hq, float *hd, int *hs, float *D, const GdArgs &G0, hipStream_t st) {
    if (!gd_fuses(s, 1) || !G0.rdy || !G0.err || G0.spin == 0) return hipErrorInvalidValue;
    const int gxg = (int)mf_cdiv((size_t)s.I, 32 * (MS_NW / 2)), gxd = (int)mf_cdiv((size_t)s.H, 32 * MS_NW);
    if ((size_t)(gxg + gxd) * (size_t)wmax >= ((size_t)1 << 31)) return hipErrorInvalidValue;
    GdArgs G = G0;
    G.need = gxg;
    const int nbH = s.nbH;
    if (nbH % MF_KC == 0 && nbH <= MS_FC * MF_KC)
        return gd_go<true, true>(layer_pl, s, wmax, work, work_n, entries, xq, xd, hq, hd, hs, D, G, gxg, gxd, st);
    if (nbH % MF_KC == 0)
        return gd_go<true, false>(layer_pl, s, wmax, work, work_n, entries, xq, xd, hq, hd, hs, D, G, gxg, gxd, st);
    return gd_go<false, false>(layer_pl, s, wmax, work, work_n, entries, xq, xd, hq, hd, hs, D, G, gxg, gxd, st);
}

}  // namespace tg
