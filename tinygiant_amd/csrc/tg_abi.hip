// tg_abi.hip -- the C ABI of libtinygiant.so (declared in include/tinygiant.h).
//
// The reference's own symbols keep their names, signatures and synchronous
// host-pointer conventions (csrc/libtinygiant.c, tinygiant/_lib.py:39-74).
// The new Q4_0 entry points run on the GPU only: every one of them checks
// for a HIP device and returns TG_E_NODEVICE rather than computing anything
// on the host.
#include "tg_internal.h"
#include "../../include/tinygiant.h"

#include <hip/hip_runtime.h>

#include <algorithm>

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>

#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <vector>

using tg::Shape;

// ================================================================ errors
static thread_local std::string g_err;

static int set_err(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define HIP_TRY(expr)                                                                      \
    do {                                                                                   \
        hipError_t e_ = (expr);                                                            \
        if (e_ != hipSuccess)                                                              \
            return set_err(TG_E_HIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_),       \
                           __FILE__, __LINE__);                                            \
    } while (0)

extern "C" const char *tg_last_error(void) { return g_err.c_str(); }

extern "C" const char *tg_version(void) { return "tinygiant-gfx950 0.1"; }

// ================================================================ device
static std::mutex g_dev_mu;
static int g_dev = -1;

static int noalloc_setup(int device);

extern "C" int tg_gpu_init(int device) {
    std::lock_guard<std::mutex> lk(g_dev_mu);
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
        return set_err(TG_E_NODEVICE, "no HIP device visible");
    if (device < 0 || device >= n) return set_err(TG_E_INVALID, "device %d out of range (0..%d)", device, n - 1);
    HIP_TRY(hipSetDevice(device));
    HIP_TRY(hipFree(nullptr));
    int rc = noalloc_setup(device);
    if (rc) return rc;
    g_dev = device;
    return TG_OK;
}

static int ensure_device() {
    if (g_dev >= 0) {
        int cur = -1;
        if (hipGetDevice(&cur) == hipSuccess && cur == g_dev) return TG_OK;
        HIP_TRY(hipSetDevice(g_dev));
        return TG_OK;
    }
    return tg_gpu_init(0);
}

extern "C" int tg_device_sync(void) {
    int rc = ensure_device();
    if (rc) return rc;
    HIP_TRY(hipDeviceSynchronize());
    return TG_OK;
}

static hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// ================================================================ timing
struct ProfRec {
    std::string kernel;
    hipEvent_t start, stop;
};
namespace tg {
thread_local LaunchEvents g_launch_ev = {nullptr, nullptr};
}
static std::mutex g_prof_mu;
static bool g_prof_on = false;
static std::vector<ProfRec> g_prof;
static std::vector<hipEvent_t> g_event_pool;

static hipEvent_t pool_event() {
    if (!g_event_pool.empty()) {
        hipEvent_t e = g_event_pool.back();
        g_event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

static void prof_clear() {
    for (auto &r : g_prof) {
        g_event_pool.push_back(r.start);
        g_event_pool.push_back(r.stop);
    }
    g_prof.clear();
}

// Records the start event of one launch; returns its slot (or -1).
// The launch inside takes the events (TG_LAUNCH), so they time the kernel's
// own execution; a launch that does not take them is timed by the start
// event recorded here and the stop event prof_end records.
static int prof_begin(const char *kernel, hipStream_t st) {
    if (!g_prof_on) return -1;
    std::lock_guard<std::mutex> lk(g_prof_mu);
    ProfRec r{kernel, pool_event(), pool_event()};
    if (!r.start || !r.stop) return -1;
    (void)hipEventRecord(r.start, st);
    g_prof.push_back(r);
    tg::g_launch_ev = {r.start, r.stop};
    return (int)g_prof.size() - 1;
}

static void prof_end(int slot, hipStream_t st) {
    if (slot < 0) return;
    std::lock_guard<std::mutex> lk(g_prof_mu);
    const bool taken = tg::g_launch_ev.start == nullptr;  // the launch recorded both events
    tg::g_launch_ev = {nullptr, nullptr};
    if (!taken) (void)hipEventRecord(g_prof[(size_t)slot].stop, st);
}

extern "C" int tg_prof_enable(int on) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    if (on) prof_clear();
    g_prof_on = on != 0;
    return TG_OK;
}

extern "C" int tg_prof_read(const char *kernel, int *launches, double *total_ms) {
    if (!kernel) return set_err(TG_E_INVALID, "kernel name is NULL");
    std::lock_guard<std::mutex> lk(g_prof_mu);
    int n = 0;
    double ms = 0.0;
    for (auto &r : g_prof) {
        if (r.kernel != kernel) continue;
        HIP_TRY(hipEventSynchronize(r.stop));
        float t = 0.0f;
        HIP_TRY(hipEventElapsedTime(&t, r.start, r.stop));
        ms += t;
        n++;
    }
    if (launches) *launches = n;
    if (total_ms) *total_ms = ms;
    return TG_OK;
}

#define PROFILED(name, st, launch)                                                             \
    do {                                                                                       \
        int slot_ = prof_begin(name, st);                                                      \
        hipError_t pe_ = (launch);                                                             \
        prof_end(slot_, st);                                                                   \
        if (pe_ != hipSuccess)                                                                 \
            return set_err(TG_E_HIP, "%s: %s (%s:%d)", #launch, hipGetErrorString(pe_), __FILE__, \
                           __LINE__);                                                          \
    } while (0)

// ================================================================ scratch
// Device memory of one MoE call beyond its inputs and outputs, for T tokens
// of one shape.  Every piece starts on a 256-byte boundary.
struct Scratch {
    float *raw = nullptr;         // T * E raw router dots
    // decode exchange words: tagged logits [T][E] u64 | tagged h blocks of
    // the fused expert launch | generation [T][2] u32 | error word; then two
    // router-partial buffers and the group hand-off words of the routed
    // one-token launch.  Tags and generations start at zero (tag 0 never
    // matches).
    uint8_t *dec = nullptr;
    size_t dec_bytes = 0;
    uint64_t *dec_lw = nullptr;
    uint64_t *dec_hw = nullptr;
    uint32_t *dec_ctl = nullptr;
    uint32_t *dec_err = nullptr;
    float *dec_part = nullptr;
    uint64_t *dec_ow = nullptr;
    uint32_t *fc_cnt = nullptr;   // arrival counts of the combine in the down launch (zero between calls)
    int32_t *ecnt = nullptr;      // E: entries placed per expert, then the arrival counts of route_q8 and of the
                                  // placing launch (zero between calls)
    int32_t *ent_cap = nullptr;   // E * T: per-expert entry lists of capacity T (chains path: over raw, unused there)
    int32_t *idx = nullptr;       // T * k
    float *w = nullptr;           // T * k
    // grouped (batched) path
    int8_t *xq = nullptr;         // T * H      Q8_0 of the normed x per token
    float *xd = nullptr;          // T * nbH
    int *xs = nullptr;            // T * nbH
    int32_t *counts = nullptr;    // E
    int32_t *offsets = nullptr;   // E + 1
    int32_t *entries = nullptr;   // T * k
    int32_t *work = nullptr;      // 2 lists x 3 * group_work_max
    int32_t *work_n = nullptr;    // 2
    int32_t *rdy = nullptr;       // group_work_max: per work item, gate/up blocks done (fused gate/up + down launch)
    int8_t *hq = nullptr;         // T * k * I  Q8_0 h per (token, slot)
    float *hd = nullptr;          // T * k * nbI
    int *hs = nullptr;            // T * k * nbI
    float *D = nullptr;           // T * k * H  down rows per (token, slot)
};

static size_t dec_words_bytes(const Shape &s, int T) {
    return 8 * ((size_t)T * s.E + tg::experts_fused_words(s)) + 8 * (size_t)T + 16;
}

// Lays the scratch of T tokens out from base (base may be null: sizes only)
// and returns its size in bytes.  The decode exchange words come first, so
// they sit at the same place for every T of one shape.
static size_t scratch_layout(const Shape &s, int T, uint8_t *base, Scratch *sc) {
    size_t off = 0;
    auto take = [&](size_t bytes) -> uint8_t * {
        const size_t o = (off + 255) & ~(size_t)255;
        off = o + bytes;
        return base ? base + o : nullptr;
    };
    const size_t n = (size_t)T * s.k;
    const size_t wmax = (size_t)tg::group_work_max(s, (int)n);
    Scratch c;
    uint8_t *dec0 = take(dec_words_bytes(s, T));
    c.dec_part = reinterpret_cast<float *>(take(4 * tg::dec_part_floats(s)));
    c.dec_ow = reinterpret_cast<uint64_t *>(take(8 * tg::dec_ow_words(s)));
    c.fc_cnt = reinterpret_cast<uint32_t *>(take(4 * tg::fuse_count_words(s, T)));
    // + the arrival counts of route_q8 and of the placing launch
    c.ecnt = reinterpret_cast<int32_t *>(take(4 * ((size_t)s.E + 2)));
    c.dec = dec0;
    c.dec_bytes = off;
    c.dec_lw = reinterpret_cast<uint64_t *>(dec0);
    c.dec_hw = c.dec_lw ? c.dec_lw + (size_t)T * s.E : nullptr;
    c.dec_ctl = c.dec_hw ? reinterpret_cast<uint32_t *>(c.dec_hw + tg::experts_fused_words(s)) : nullptr;
    c.dec_err = c.dec_ctl ? c.dec_ctl + 2 * (size_t)T : nullptr;
    c.raw = reinterpret_cast<float *>(take(4 * (size_t)T * s.E));
    c.idx = reinterpret_cast<int32_t *>(take(4 * n));
    c.w = reinterpret_cast<float *>(take(4 * n));
    c.xq = reinterpret_cast<int8_t *>(take((size_t)T * s.H));
    c.xd = reinterpret_cast<float *>(take(4 * (size_t)T * s.nbH));
    c.xs = reinterpret_cast<int *>(take(4 * (size_t)T * s.nbH));
    c.counts = reinterpret_cast<int32_t *>(take(4 * (size_t)s.E));
    c.offsets = reinterpret_cast<int32_t *>(take(4 * ((size_t)s.E + 1)));
    c.entries = reinterpret_cast<int32_t *>(take(4 * n));
    c.ent_cap = reinterpret_cast<int32_t *>(c.raw);  // T * E words, like the router dots the chains path leaves unused
    c.hq = reinterpret_cast<int8_t *>(take(n * s.I));
    c.hd = reinterpret_cast<float *>(take(4 * n * s.nbI));
    c.hs = reinterpret_cast<int *>(take(4 * n * s.nbI));
    c.D = reinterpret_cast<float *>(take(4 * n * s.H));
    c.work = reinterpret_cast<int32_t *>(take(4 * 2 * 3 * wmax));
    c.work_n = reinterpret_cast<int32_t *>(take(4 * 2));
    c.rdy = reinterpret_cast<int32_t *>(take(4 * wmax));
    if (sc) *sc = c;
    return (off + 255) & ~(size_t)255;
}

// ================================================================ arena
struct tg_arena {
    Shape s;
    int L = 0;
    uint8_t *experts = nullptr;   // L * LB bytes, tensor-planar per tensor
    float *routers = nullptr;     // L * E * H, the router as loaded times the norm weight (per column)
    float *routers_raw = nullptr; // L * E * H, the router as loaded
    float *norms = nullptr;       // L * H, FFN norm weight (ones until loaded)
    uint8_t *staging = nullptr;   // LB bytes, relayout form for load/read
    // per-call scratch, grown on demand (one allocation, laid out by
    // scratch_layout), and the host-pointer entry points' x / out buffers
    int cap_T = 0;
    uint8_t *sc_mem = nullptr;
    Scratch sc;
    float *xbuf = nullptr;        // T * H (host-pointer entry points)
    float *obuf = nullptr;        // T * H
    int batch_path = TG_BATCH_AUTO;
    // captured stacks, replayed as HIP graphs
    struct Graph {
        const float *x;
        int T, layer0, n;
        float eps;
        hipGraph_t graph;
        hipGraphExec_t exec;
    };
    std::vector<Graph> graphs;
    hipStream_t capture = nullptr;
    bool use_graphs = false;  // stack calls replayed as graphs (tg_arena_set_graphs)
    int decode_path = TG_DECODE_AUTO;
    int n_cu = 0;
};

static bool graphs_default();

static void drop_graphs(tg_arena *a) {
    for (auto &g : a->graphs) {
        (void)hipGraphExecDestroy(g.exec);
        (void)hipGraphDestroy(g.graph);
    }
    a->graphs.clear();
}

static int check_shape(int H, int I, int E, int k) {
    if (H <= 0 || I <= 0 || H % 256 || I % 32)
        return set_err(TG_E_INVALID, "embed_dim must be a positive multiple of 256 and inter_dim of 32 (got %d, %d)",
                       H, I);
    if (H / 32 > tg::MAX_NB || I / 32 > tg::MAX_NB)
        return set_err(TG_E_INVALID, "embed_dim / inter_dim above %d", tg::MAX_NB * 32);
    if (E <= 0 || E > tg::MAX_E - 4 || E % 4)
        return set_err(TG_E_INVALID, "n_experts must be a multiple of 4 in 4..%d (got %d)", tg::MAX_E - 4, E);
    if (k <= 0 || k > tg::MAX_K || k > E)
        return set_err(TG_E_INVALID, "top_k must be in 1..min(%d, n_experts) (got %d)", tg::MAX_K, k);
    return TG_OK;
}

static void dfree(void *p) {
    if (p) (void)hipFree(p);
}

static void arena_free(tg_arena *a) {
    if (!a) return;
    drop_graphs(a);
    if (a->capture) (void)hipStreamDestroy(a->capture);
    dfree(a->experts);
    dfree(a->routers);
    dfree(a->routers_raw);
    dfree(a->norms);
    dfree(a->staging);
    dfree(a->sc_mem);
    dfree(a->xbuf);
    dfree(a->obuf);
    delete a;
}

extern "C" tg_arena *tg_arena_create(int n_layers, int n_experts, int embed_dim, int inter_dim, int top_k) {
    if (n_layers <= 0) { set_err(TG_E_INVALID, "n_layers must be positive"); return nullptr; }
    if (check_shape(embed_dim, inter_dim, n_experts, top_k)) return nullptr;
    tg::Shape shape = tg::make_shape(embed_dim, inter_dim, n_experts, top_k);
    if (!tg::decode_shape_ok(shape)) {
        set_err(TG_E_INVALID, "shape H=%d I=%d E=%d k=%d exceeds the decode kernels' limits", embed_dim, inter_dim,
                n_experts, top_k);
        return nullptr;
    }
    if (ensure_device()) return nullptr;
    tg_arena *a = new tg_arena();
    a->s = shape;
    a->L = n_layers;
    a->use_graphs = graphs_default();
    {
        int dev = 0, v = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess) a->n_cu = v;
    }
    size_t eb = a->s.LB * (size_t)n_layers;
    size_t rb = sizeof(float) * (size_t)n_experts * embed_dim * n_layers;
    size_t nb = sizeof(float) * (size_t)embed_dim * n_layers;
    if (hipMalloc(&a->experts, eb) != hipSuccess || hipMalloc(&a->routers, rb) != hipSuccess ||
        hipMalloc(&a->routers_raw, rb) != hipSuccess || hipMalloc(&a->norms, nb) != hipSuccess) {
        (void)hipGetLastError();
        set_err(TG_E_NOMEM, "hipMalloc of %.2f GB expert arena failed", (eb + 2 * rb + nb) / 1e9);
        arena_free(a);
        return nullptr;
    }
    // unit norm weight until tg_arena_load_norm
    if (tg::launch_fill(a->norms, 1.0f, (size_t)embed_dim * n_layers, nullptr) != hipSuccess ||
        hipStreamSynchronize(nullptr) != hipSuccess) {
        set_err(TG_E_HIP, "initialising the norm weights failed");
        arena_free(a);
        return nullptr;
    }
    return a;
}

extern "C" void tg_arena_destroy(tg_arena *a) { arena_free(a); }

extern "C" size_t tg_arena_expert_bytes(const tg_arena *a) { return a ? a->s.EB : 0; }
extern "C" size_t tg_arena_layer_bytes(const tg_arena *a) { return a ? a->s.LB : 0; }

extern "C" int tg_arena_expert_offset(const tg_arena *a, int expert, size_t *offset, size_t *gate_bytes,
                                      size_t *up_bytes, size_t *down_bytes) {
    if (!a) return set_err(TG_E_INVALID, "arena is NULL");
    if (expert < 0 || expert >= a->s.E) return set_err(TG_E_INVALID, "expert %d out of range", expert);
    if (offset) *offset = (size_t)expert * a->s.EB;
    if (gate_bytes) *gate_bytes = a->s.GB;
    if (up_bytes) *up_bytes = a->s.GB;
    if (down_bytes) *down_bytes = a->s.DB;
    return TG_OK;
}

static int arena_layer_check(tg_arena *a, int layer) {
    if (!a) return set_err(TG_E_INVALID, "arena is NULL");
    if (layer < 0 || layer >= a->L) return set_err(TG_E_INVALID, "layer %d out of range 0..%d", layer, a->L - 1);
    return ensure_device();
}

static int arena_staging(tg_arena *a) {
    if (a->staging) return TG_OK;
    if (hipMalloc(&a->staging, a->s.LB) != hipSuccess) {
        (void)hipGetLastError();
        return set_err(TG_E_NOMEM, "hipMalloc of %zu-byte staging buffer failed", a->s.LB);
    }
    return TG_OK;
}

extern "C" int tg_arena_load_layer(tg_arena *a, int layer, const void *host_bytes, size_t nbytes) {
    int rc = arena_layer_check(a, layer);
    if (rc) return rc;
    if (!host_bytes) return set_err(TG_E_INVALID, "host_bytes is NULL");
    if (nbytes != a->s.LB) return set_err(TG_E_INVALID, "layer file has %zu bytes, expected %zu", nbytes, a->s.LB);
    if ((rc = arena_staging(a))) return rc;
    HIP_TRY(hipMemcpy(a->staging, host_bytes, nbytes, hipMemcpyHostToDevice));
    HIP_TRY(tg::launch_repack_layer(a->staging, a->experts + (size_t)layer * a->s.LB, a->s, true, nullptr));
    HIP_TRY(hipStreamSynchronize(nullptr));
    return TG_OK;
}

extern "C" int tg_arena_read_layer(tg_arena *a, int layer, void *host_bytes, size_t nbytes) {
    int rc = arena_layer_check(a, layer);
    if (rc) return rc;
    if (!host_bytes) return set_err(TG_E_INVALID, "host_bytes is NULL");
    if (nbytes != a->s.LB) return set_err(TG_E_INVALID, "buffer has %zu bytes, expected %zu", nbytes, a->s.LB);
    if ((rc = arena_staging(a))) return rc;
    HIP_TRY(tg::launch_repack_layer(a->experts + (size_t)layer * a->s.LB, a->staging, a->s, false, nullptr));
    HIP_TRY(hipMemcpy(host_bytes, a->staging, nbytes, hipMemcpyDeviceToHost));
    return TG_OK;
}

extern "C" int tg_arena_read_expert(tg_arena *a, int layer, int expert, void *host_bytes, size_t nbytes) {
    int rc = arena_layer_check(a, layer);
    if (rc) return rc;
    const Shape &s = a->s;
    if (expert < 0 || expert >= s.E) return set_err(TG_E_INVALID, "expert %d out of range 0..%d", expert, s.E - 1);
    if (!host_bytes) return set_err(TG_E_INVALID, "host_bytes is NULL");
    if (nbytes != s.EB) return set_err(TG_E_INVALID, "buffer has %zu bytes, expected %zu", nbytes, s.EB);
    if ((rc = arena_staging(a))) return rc;
    // gate, up and down are planar each: three tensors back to the relayout blocks
    const uint8_t *src = a->experts + (size_t)layer * s.LB + (size_t)expert * s.EB;
    const size_t gblk = (size_t)s.I * s.nbH, dblk = (size_t)s.H * s.nbI;
    HIP_TRY(tg::launch_repack_tensor(src, a->staging, gblk, false, nullptr));
    HIP_TRY(tg::launch_repack_tensor(src + s.GB, a->staging + s.GB, gblk, false, nullptr));
    HIP_TRY(tg::launch_repack_tensor(src + 2 * s.GB, a->staging + 2 * s.GB, dblk, false, nullptr));
    HIP_TRY(hipMemcpy(host_bytes, a->staging, nbytes, hipMemcpyDeviceToHost));
    return TG_OK;
}

static const float *norm_of(const tg_arena *a, int layer) { return a->norms + (size_t)layer * a->s.H; }

// The kernels use router * g (per column), recomputed from the router as
// loaded whenever either changes.
static int arena_refresh_router(tg_arena *a, int layer) {
    const size_t n = (size_t)a->s.E * a->s.H;
    HIP_TRY(tg::launch_scale_router(a->routers_raw + (size_t)layer * n, norm_of(a, layer),
                                    a->routers + (size_t)layer * n, a->s.E, a->s.H, nullptr));
    HIP_TRY(hipStreamSynchronize(nullptr));
    return TG_OK;
}

extern "C" int tg_arena_load_router(tg_arena *a, int layer, const float *host_router, size_t count) {
    int rc = arena_layer_check(a, layer);
    if (rc) return rc;
    size_t n = (size_t)a->s.E * a->s.H;
    if (!host_router || count != n) return set_err(TG_E_INVALID, "router needs %zu floats (got %zu)", n, count);
    HIP_TRY(hipMemcpy(a->routers_raw + (size_t)layer * n, host_router, n * sizeof(float), hipMemcpyHostToDevice));
    return arena_refresh_router(a, layer);
}

extern "C" int tg_arena_load_norm(tg_arena *a, int layer, const float *host_norm, size_t count) {
    int rc = arena_layer_check(a, layer);
    if (rc) return rc;
    const size_t n = (size_t)a->s.H;
    if (!host_norm || count != n) return set_err(TG_E_INVALID, "norm weight needs %zu floats (got %zu)", n, count);
    HIP_TRY(hipMemcpy(a->norms + (size_t)layer * n, host_norm, n * sizeof(float), hipMemcpyHostToDevice));
    return arena_refresh_router(a, layer);
}

extern "C" int tg_arena_synth_layer(tg_arena *a, int layer, uint64_t seed, float sigma) {
    int rc = arena_layer_check(a, layer);
    if (rc) return rc;
    HIP_TRY(tg::launch_synth_layer(a->experts + (size_t)layer * a->s.LB,
                                   a->routers_raw + (size_t)layer * a->s.E * a->s.H, a->s, layer, seed, sigma,
                                   nullptr));
    return arena_refresh_router(a, layer);
}

static int arena_scratch(tg_arena *a, int T) {
    if (T <= a->cap_T) return TG_OK;
    drop_graphs(a);  // captured graphs point at the old buffers
    dfree(a->sc_mem); dfree(a->xbuf); dfree(a->obuf);
    a->sc_mem = nullptr; a->xbuf = nullptr; a->obuf = nullptr;
    a->sc = Scratch();
    a->cap_T = 0;
    const Shape &s = a->s;
    const size_t bytes = scratch_layout(s, T, nullptr, nullptr);
    bool ok = hipMalloc(&a->sc_mem, bytes) == hipSuccess &&
              hipMalloc(&a->xbuf, sizeof(float) * (size_t)T * s.H) == hipSuccess &&
              hipMalloc(&a->obuf, sizeof(float) * (size_t)T * s.H) == hipSuccess;
    if (ok) {
        scratch_layout(s, T, a->sc_mem, &a->sc);
        ok = hipMemset(a->sc_mem, 0, a->sc.dec_bytes) == hipSuccess;  // tags and generations start at zero
    }
    if (!ok) {
        (void)hipGetLastError();
        return set_err(TG_E_NOMEM, "scratch for %d tokens", T);
    }
    a->cap_T = T;
    return TG_OK;
}

// ================================================================ MoE block
static const float *router_of(tg_arena *a, int layer) {
    return a->routers + (size_t)layer * a->s.E * a->s.H;
}

// One MoE block: raw router dots, gate/up (norm, routing and Q8_0 fused),
// down + combine.  out = moe_out (resid NULL) or resid + moe_out.
static bool grouped_usable(tg_arena *a, int T) {
    if (a->batch_path == TG_BATCH_PER_TOKEN) return false;
    if (a->batch_path == TG_BATCH_GROUPED || a->batch_path == TG_BATCH_GROUPED_DOT) return tg::grouped_shape_ok(a->s);
    return T >= 2 && tg::grouped_shape_ok(a->s);
}

// The MFMA kernels address activation rows with 32-bit offsets.
static bool mfma_usable(tg_arena *a, int T) {
    const Shape &s = a->s;
    const size_t span = (size_t)T * s.k * (size_t)(s.H > s.I ? s.H : s.I);
    return a->batch_path != TG_BATCH_GROUPED_DOT && tg::mfma_shape_ok(s) && span < (size_t)INT32_MAX;
}

// One MoE block over T tokens grouped by expert: every selected expert's
// weights stream once for all its tokens.
static int layer_kernels_grouped(tg_arena *a, const Scratch &c, int layer, const float *x, float *out, const float *resid, int T,
                                 float eps, hipStream_t st) {
    const Shape &s = a->s;
    const uint8_t *lp = a->experts + (size_t)layer * s.LB;
    // few tokens: the router's group chains go to the down rows' buffer (free
    // until the down kernel; G T E <= T k H floats when E <= 32 k) and
    // route_q8 adds them; otherwise the router dots
    const bool chains = tg::route_chains_usable(T, s.E, s.H) && (size_t)s.E <= 32 * (size_t)s.k;
    if (chains)
        PROFILED("route", st, tg::launch_route_chains(router_of(a, layer), x, T, s.E, s.H, c.D, st));
    else
        PROFILED("route", st, tg::launch_route(router_of(a, layer), x, T, s.E, s.H, c.raw, st));
    // MFMA path with few tokens: route_q8 also places each entry in its
    // expert's list (capacity T), so the grouping kernel only builds the work
    // items (from 128 tokens the placement's global atomics, about 16 per
    // expert per 128 tokens on one counter, cost more than the grouping kernel
    // saves: 2048 tokens, route_q8 10.6 -> 32.4 us for group 12.6 -> 7.1 us)
    const bool mfma = mfma_usable(a, T), placed = mfma && chains;
    const int n = T * s.k;
    const int mt = mfma ? tg::mfma_tiles(s, T) : 0, ch = mfma ? tg::mfma_item_entries(s, mt) : 0;
    const int wmax = mfma ? tg::group_work_max(s, n, ch) : 0;
    // gate/up and down in one launch where the one-tile kernels take it
    // (the combine stays a launch of its own)
    const bool gd = mfma && tg::gd_fuses(s, mt) && !tg::down_fuses(s, mt, T) && wmax <= tg::group_work_max(s, n);
    const bool gd16 =
        mfma && !gd && tg::gd16_fuses(s, mt) && !tg::down_fuses(s, mt, T) && wmax <= tg::group_work_max(s, n);
    int32_t *rdy = gd || gd16 ? c.rdy : nullptr;
    // one-tile items over the placed lists: the last route_q8 block builds
    // the work items (no grouping launch)
    tg::RouteGroup rg;
    const bool q8_groups = placed && ch <= 32 && tg::route_groups_on();
    if (q8_groups) {
        rg.counts = c.counts;
        rg.offsets = c.offsets;
        rg.work = c.work;
        rg.work_n = c.work_n;
        rg.rdy = rdy;
        rg.arrive = reinterpret_cast<uint32_t *>(c.ecnt + s.E);
        rg.ch = ch;
        rg.wmax = wmax;
    }
    PROFILED("route_q8", st,
             tg::launch_route_q8(c.raw, chains ? c.D : nullptr, x, norm_of(a, layer), T, s.E, s.H, s.k, eps, c.idx,
                                 c.w, c.xq, c.xd, c.xs, placed ? c.ecnt : nullptr, placed ? c.ent_cap : nullptr, rg,
                                 st));
    if (mfma) {
        // many entries: placed by many blocks into the lists over the
        // router-dot buffer (route_q8 has read it), then only the work items
        const bool par = !placed && tg::place_par_on();
        int32_t *ent = placed || par ? c.ent_cap : c.entries;
        if (par) {
            tg::RouteGroup pg;
            pg.counts = c.counts;
            pg.offsets = c.offsets;
            pg.work = c.work;
            pg.work_n = c.work_n;
            pg.rdy = rdy;
            pg.arrive = reinterpret_cast<uint32_t *>(c.ecnt + s.E + 1);
            pg.ch = ch;
            pg.wmax = wmax;
            PROFILED("group", st, tg::launch_place(c.idx, n, s.E, T, c.ecnt, c.ent_cap, pg, st));
        } else if (!q8_groups && placed)
            PROFILED("group", st,
                     tg::launch_group_placed(s, n, ch, T, c.ecnt, c.counts, c.offsets, c.work, c.work_n, rdy, st));
        else if (!q8_groups)
            PROFILED("group", st,
                     tg::launch_group_chunked(s, c.idx, n, ch, c.counts, c.offsets, c.entries, c.work, c.work_n,
                                              rdy, st));
        if (gd || gd16) {
            tg::GdArgs G;
            G.rdy = c.rdy;
            G.err = c.dec_err;
            G.spin = tg::poll_spin_limit();
            G.drop = tg::poll_drop();
            if (gd)
                PROFILED("gu_down_mfma", st,
                         tg::launch_gu_down_ms(lp, s, wmax, c.work, c.work_n, ent, c.xq, c.xd, c.hq, c.hd, c.hs, c.D,
                                               G, st));
            else
                PROFILED("gu_down_mfma", st,
                         tg::launch_gu_down_x16(lp, s, wmax, c.work, c.work_n, ent, c.xq, c.xd, c.hq, c.hd, c.hs,
                                                c.D, G, st));
            PROFILED("combine", st, tg::launch_combine(c.D, c.w, T, s.H, s.k, resid, out, st));
            return TG_OK;
        }
        PROFILED("gateup_mfma", st,
                 tg::launch_gateup_mfma(lp, s, mt, wmax, c.work, c.work_n, ent, c.xq, c.xd, c.xs, c.hq, c.hd, c.hs,
                                        st));
        // the combine inside the down launch where its kernel takes it
        tg::FuseArgs F;
        const bool fuse = tg::down_fuses(s, mt, T);
        if (fuse) {
            F.w = c.w;
            F.resid = resid;
            F.out = out;
            F.cnt = c.fc_cnt;
        }
        PROFILED("down_mfma", st,
                 tg::launch_down_mfma(lp, s, mt, wmax, c.work, c.work_n, ent, c.hq, c.hd, c.hs, c.D, F, st));
        if (!fuse) PROFILED("combine", st, tg::launch_combine(c.D, c.w, T, s.H, s.k, resid, out, st));
        return TG_OK;
    }
    PROFILED("group", st,
             tg::launch_group(s, c.idx, n, c.counts, c.offsets, c.entries, c.work, c.work_n, st));
    PROFILED("gateup_grouped", st,
             tg::launch_gateup_grouped(lp, s, n, c.work, c.work_n, c.entries, c.xq, c.xd, c.xs, c.hq, c.hd,
                                       c.hs, st));
    PROFILED("down_grouped", st,
             tg::launch_down_grouped(lp, s, n, c.work, c.work_n, c.entries, c.hq, c.hd, c.hs, c.D, st));
    PROFILED("combine", st, tg::launch_combine(c.D, c.w, T, s.H, s.k, resid, out, st));
    return TG_OK;
}

// One token, one launch per layer that also routes (the default one-token
// path where the shape allows it).
static bool routed_usable(tg_arena *a, int T) {
    return T == 1 && (a->decode_path == TG_DECODE_AUTO || a->decode_path == TG_DECODE_ROUTED) &&
           tg::layer_dec_ok(a->s, a->n_cu);
}

// One token, gate/up and down in one launch after a routing kernel.
static bool fused_usable(tg_arena *a, int T) {
    return T == 1 && (a->decode_path == TG_DECODE_AUTO || a->decode_path == TG_DECODE_FUSED) &&
           tg::experts_fused_ok(a->s, a->n_cu);
}

// Layers [l0, l0 + n) of one token on the routed path: the prologue forms the
// first layer's router partials and reserves one generation per layer; layer
// j reads the partials buffer j % 2 and leaves the next layer's in the
// other.  Layer j's top-k ids / weights go to idx + j * k_step (k_step 0:
// every layer overwrites the same k entries).
static int routed_layers(tg_arena *a, const Scratch &c, int l0, int n, const float *x, float *out, const float *resid, float eps,
                         int32_t *idx, float *w, int k_step, hipStream_t st) {
    const Shape &s = a->s;
    const size_t half = tg::dec_part_floats(s) / 2;
    PROFILED("dec_part", st, tg::launch_dec_part(router_of(a, l0), x, s, c.dec_part, c.dec_ctl, n, st));
    for (int j = 0; j < n; j++) {
        const int l = l0 + j;
        const float *wr_next = j + 1 < n ? router_of(a, l + 1) : nullptr;
        PROFILED("layer", st,
                 tg::launch_layer_dec(a->experts + (size_t)l * s.LB, s, a->n_cu, j == 0 ? x : out, norm_of(a, l),
                                      c.dec_part + (size_t)(j & 1) * half, wr_next,
                                      c.dec_part + (size_t)((j + 1) & 1) * half, c.dec_hw, c.dec_ow, c.dec_ctl,
                                      (uint32_t)(n - 1 - j), c.dec_err, j == 0 ? resid : out, out,
                                      idx + (size_t)j * k_step, w + (size_t)j * k_step, eps, st));
    }
    return TG_OK;
}

static int layer_kernels(tg_arena *a, const Scratch &c, int layer, const float *x, float *out, const float *resid, int T, float eps,
                         hipStream_t st) {
    if (grouped_usable(a, T)) return layer_kernels_grouped(a, c, layer, x, out, resid, T, eps, st);
    if (routed_usable(a, T)) return routed_layers(a, c, layer, 1, x, out, resid, eps, c.idx, c.w, 0, st);
    const Shape &s = a->s;
    const uint8_t *lp = a->experts + (size_t)layer * s.LB;
    PROFILED("route", st,
             tg::launch_route_dec(router_of(a, layer), x, norm_of(a, layer), T, s, eps, c.dec_lw, c.dec_ctl,
                                  c.dec_err, c.idx, c.w, c.xq, c.xd, c.xs, st));
    if (fused_usable(a, T)) {
        PROFILED("experts", st,
                 tg::launch_experts_fused(lp, s, a->n_cu, c.idx, c.w, c.xq, c.xd, c.xs, c.dec_hw, c.dec_ctl,
                                          c.dec_err, resid, out, st));
        return TG_OK;
    }
    PROFILED("gateup", st, tg::launch_gateup(lp, s, T, c.idx, c.xq, c.xd, c.xs, c.hq, c.hd, c.hs, st));
    PROFILED("down", st, tg::launch_down(lp, s, T, c.idx, c.w, c.hq, c.hd, c.hs, resid, out, st));
    return TG_OK;
}

static int moe_layer_launch(tg_arena *a, const Scratch &c, int layer, const float *x, float *out, const float *resid, int T,
                            int32_t *idx_out, float *w_out, float eps, hipStream_t st) {
    const Shape &s = a->s;
    int rc = layer_kernels(a, c, layer, x, out, resid, T, eps, st);
    if (rc) return rc;
    if (idx_out) HIP_TRY(hipMemcpyAsync(idx_out, c.idx, sizeof(int32_t) * (size_t)T * s.k, hipMemcpyDeviceToDevice, st));
    if (w_out) HIP_TRY(hipMemcpyAsync(w_out, c.w, sizeof(float) * (size_t)T * s.k, hipMemcpyDeviceToDevice, st));
    return TG_OK;
}

// x <- x + MoE_l(x) for layers [l0, l0+n), in place.
static int stack_launch(tg_arena *a, const Scratch &c, float *x, int T, int l0, int n, float eps, hipStream_t st) {
    if (routed_usable(a, T)) return routed_layers(a, c, l0, n, x, x, x, eps, c.idx, c.w, 0, st);
    for (int l = l0; l < l0 + n; l++) {
        int rc = layer_kernels(a, c, l, x, x, x, T, eps, st);
        if (rc) return rc;
    }
    return TG_OK;
}

// the default of new arenas: direct launches unless TG_GRAPH=1
static bool graphs_default() {
    static const bool on = [] {
        const char *e = getenv("TG_GRAPH");
        return e && e[0] == '1';
    }();
    return on;
}

// A stack call is launched layer by layer (the default, and always while
// kernel timing is on), or, with graphs on, replayed as a HIP graph captured
// on first use for this (x, T, layer range, eps).
static int stack_run(tg_arena *a, float *x, int T, int l0, int n, float eps, hipStream_t st) {
    if (!a->use_graphs || g_prof_on) return stack_launch(a, a->sc, x, T, l0, n, eps, st);
    for (auto &g : a->graphs)
        if (g.x == x && g.T == T && g.layer0 == l0 && g.n == n && g.eps == eps) {
            HIP_TRY(hipGraphLaunch(g.exec, st));
            return TG_OK;
        }
    if (!a->capture) HIP_TRY(hipStreamCreateWithFlags(&a->capture, hipStreamNonBlocking));
    tg_arena::Graph g{x, T, l0, n, eps, nullptr, nullptr};
    HIP_TRY(hipStreamBeginCapture(a->capture, hipStreamCaptureModeRelaxed));
    int rc = stack_launch(a, a->sc, x, T, l0, n, eps, a->capture);
    hipError_t ec = hipStreamEndCapture(a->capture, &g.graph);
    if (rc) return rc;
    if (ec != hipSuccess) return set_err(TG_E_HIP, "graph capture failed: %s", hipGetErrorString(ec));
    ec = hipGraphInstantiate(&g.exec, g.graph, nullptr, nullptr, 0);
    if (ec != hipSuccess) {
        (void)hipGraphDestroy(g.graph);
        return set_err(TG_E_HIP, "graph instantiate failed: %s", hipGetErrorString(ec));
    }
    if (a->graphs.size() >= 8) {
        (void)hipGraphExecDestroy(a->graphs.front().exec);
        (void)hipGraphDestroy(a->graphs.front().graph);
        a->graphs.erase(a->graphs.begin());
    }
    a->graphs.push_back(g);
    HIP_TRY(hipGraphLaunch(g.exec, st));
    return TG_OK;
}

extern "C" int tg_arena_status(tg_arena *a);

static int check_tokens(int T) {
    if (T <= 0 || T > 65535) return set_err(TG_E_INVALID, "n_tokens must be in 1..65535 (got %d)", T);
    return TG_OK;
}

extern "C" int tg_moe_layer_q40_dev(tg_arena *a, int layer, const float *x, float *moe_out, int n_tokens,
                                    int32_t *topk_idx, float *topk_w, float eps, void *stream) {
    int rc = arena_layer_check(a, layer);
    if (rc) return rc;
    if ((rc = check_tokens(n_tokens))) return rc;
    if (!x || !moe_out) return set_err(TG_E_INVALID, "x / moe_out is NULL");
    if ((rc = arena_scratch(a, n_tokens))) return rc;
    return moe_layer_launch(a, a->sc, layer, x, moe_out, nullptr, n_tokens, topk_idx, topk_w, eps, as_stream(stream));
}

extern "C" int tg_moe_layer_q40(tg_arena *a, int layer, const float *x, float *moe_out, int n_tokens,
                                int32_t *topk_idx, float *topk_w, float eps) {
    int rc = arena_layer_check(a, layer);
    if (rc) return rc;
    if ((rc = check_tokens(n_tokens))) return rc;
    if (!x || !moe_out) return set_err(TG_E_INVALID, "x / moe_out is NULL");
    if ((rc = arena_scratch(a, n_tokens))) return rc;
    const Shape &s = a->s;
    size_t nx = (size_t)n_tokens * s.H;
    HIP_TRY(hipMemcpy(a->xbuf, x, nx * sizeof(float), hipMemcpyHostToDevice));
    if ((rc = moe_layer_launch(a, a->sc, layer, a->xbuf, a->obuf, nullptr, n_tokens, nullptr, nullptr, eps, nullptr)))
        return rc;
    HIP_TRY(hipMemcpy(moe_out, a->obuf, nx * sizeof(float), hipMemcpyDeviceToHost));
    if (topk_idx) HIP_TRY(hipMemcpy(topk_idx, a->sc.idx, sizeof(int32_t) * (size_t)n_tokens * s.k, hipMemcpyDeviceToHost));
    if (topk_w) HIP_TRY(hipMemcpy(topk_w, a->sc.w, sizeof(float) * (size_t)n_tokens * s.k, hipMemcpyDeviceToHost));
    return tg_arena_status(a);  // a poll that ran out of tries (its rows are NaN)
}

static int stack_check(tg_arena *a, int layer0, int n_layers, int T, const float *x) {
    if (!a) return set_err(TG_E_INVALID, "arena is NULL");
    if (n_layers <= 0 || layer0 < 0 || layer0 + n_layers > a->L)
        return set_err(TG_E_INVALID, "layers %d..%d outside the arena's %d", layer0, layer0 + n_layers - 1, a->L);
    int rc = check_tokens(T);
    if (rc) return rc;
    if (!x) return set_err(TG_E_INVALID, "x is NULL");
    if ((rc = ensure_device())) return rc;
    return arena_scratch(a, T);
}

extern "C" int tg_moe_stack_q40_dev(tg_arena *a, float *x, int n_tokens, int layer0, int n_layers, float eps,
                                    void *stream) {
    int rc = stack_check(a, layer0, n_layers, n_tokens, x);
    if (rc) return rc;
    return stack_run(a, x, n_tokens, layer0, n_layers, eps, as_stream(stream));
}

extern "C" int tg_moe_stack_q40_trace_dev(tg_arena *a, float *x, int layer0, int n_layers, float eps,
                                          int32_t *topk_idx, float *topk_w, void *stream) {
    int rc = stack_check(a, layer0, n_layers, 1, x);
    if (rc) return rc;
    if (!topk_idx || !topk_w) return set_err(TG_E_INVALID, "topk_idx / topk_w is NULL");
    hipStream_t st = as_stream(stream);
    const size_t k = (size_t)a->s.k;
    if (routed_usable(a, 1)) return routed_layers(a, a->sc, layer0, n_layers, x, x, x, eps, topk_idx, topk_w, (int)k, st);
    for (int l = 0; l < n_layers; l++) {
        if ((rc = layer_kernels(a, a->sc, layer0 + l, x, x, x, 1, eps, st))) return rc;
        HIP_TRY(hipMemcpyAsync(topk_idx + l * k, a->sc.idx, sizeof(int32_t) * k, hipMemcpyDeviceToDevice, st));
        HIP_TRY(hipMemcpyAsync(topk_w + l * k, a->sc.w, sizeof(float) * k, hipMemcpyDeviceToDevice, st));
    }
    return TG_OK;
}

extern "C" int tg_arena_set_graphs(tg_arena *a, int on) {
    if (!a) return set_err(TG_E_INVALID, "arena is NULL");
    drop_graphs(a);
    a->use_graphs = on != 0;
    return TG_OK;
}

extern "C" int tg_arena_set_batch_path(tg_arena *a, int path) {
    if (!a) return set_err(TG_E_INVALID, "arena is NULL");
    if (path != TG_BATCH_AUTO && path != TG_BATCH_GROUPED && path != TG_BATCH_PER_TOKEN &&
        path != TG_BATCH_GROUPED_DOT)
        return set_err(TG_E_INVALID, "unknown batch path %d", path);
    if ((path == TG_BATCH_GROUPED || path == TG_BATCH_GROUPED_DOT) && !tg::grouped_shape_ok(a->s))
        return set_err(TG_E_UNSUPPORTED, "the grouped path is not available for this shape");
    drop_graphs(a);  // captured graphs hold the previous path's kernels
    a->batch_path = path;
    return TG_OK;
}

extern "C" int tg_arena_set_decode_path(tg_arena *a, int path) {
    if (!a) return set_err(TG_E_INVALID, "arena is NULL");
    if (path != TG_DECODE_AUTO && path != TG_DECODE_PER_LAYER && path != TG_DECODE_FUSED &&
        path != TG_DECODE_ROUTED)
        return set_err(TG_E_INVALID, "unknown decode path %d", path);
    if (path == TG_DECODE_FUSED && !tg::experts_fused_ok(a->s, a->n_cu))
        return set_err(TG_E_UNSUPPORTED, "the fused expert launch is not available for this shape");
    if (path == TG_DECODE_ROUTED && !tg::layer_dec_ok(a->s, a->n_cu))
        return set_err(TG_E_UNSUPPORTED, "the routed one-token launch is not available for this shape");
    drop_graphs(a);
    a->decode_path = path;
    return TG_OK;
}

// ================================================================ no-alloc layer call
// tg_moe_layer_q40_noalloc_dev runs tg_moe_layer_q40_dev's kernels with
// their scratch in `scratch`, a fixed device array (each GPU holds its own
// copy until the process ends), so the call allocates nothing.  In host code
// the array's name is not a device address: each device's address comes
// from hipGetSymbolAddress at set-up (tg_gpu_init, with that device
// current) and only that address is used.
//
// The array keeps the last call's contents.  It starts with a 256-byte
// header: the layout key of the words behind it (8 bytes) and the error word
// of the one-token launches (4 bytes).  Behind it every call of one shape
// uses the same layout, the scratch of the largest token count that fits, so
// calls with different token counts share their tagged exchange words and
// generations.  Those must start at zero for a layout: each call first runs
// a one-block kernel that compares the header's key with the call's shape
// and, when they differ, clears the exchange words and stores the key.  The
// decision is taken on the device, so it holds for calls replayed from a
// captured graph as well as for direct ones.  Calls that overlap on one
// device race.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)16 << 20;
constexpr size_t NOALLOC_HEADER = 256;
constexpr int NOALLOC_MAX_DEV = 64;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

struct NoAllocDev {
    uint8_t *ptr = nullptr;  // this device's copy of `scratch`
    bool used = false;       // a call has run on it since set-up
};
static std::mutex g_na_mu;
static NoAllocDev g_na[NOALLOC_MAX_DEV];

// With `device` current: its address of the array.
static int noalloc_setup(int device) {
    if (device < 0 || device >= NOALLOC_MAX_DEV) return TG_OK;  // the no-alloc call refuses such devices
    std::lock_guard<std::mutex> lk(g_na_mu);
    if (g_na[device].ptr) return TG_OK;
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return set_err(TG_E_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
    g_na[device].ptr = static_cast<uint8_t *>(p);
    return TG_OK;
}

static uint64_t noalloc_key(const Shape &s) {
    return (1ull << 63) | ((uint64_t)s.H << 40) | ((uint64_t)s.I << 20) | ((uint64_t)s.E << 8) | (uint64_t)s.k;
}

// The largest token count whose scratch fits behind the header (0: none).
static int noalloc_tmax(const Shape &s) {
    const size_t room = NOALLOC_SCRATCH_BYTES - NOALLOC_HEADER;
    int lo = 0, hi = 65535;
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (scratch_layout(s, mid, nullptr, nullptr) <= room)
            lo = mid;
        else
            hi = mid - 1;
    }
    return lo;
}

static uint32_t *noalloc_err(uint8_t *base) { return reinterpret_cast<uint32_t *>(base + 8); }

extern "C" int tg_moe_layer_q40_noalloc_dev(tg_arena *a, int layer, const float *x, float *moe_out, int n_tokens,
                                            int32_t *topk_idx, float *topk_w, float eps, void *stream) {
    if (!a) return set_err(TG_E_INVALID, "arena is NULL");
    if (layer < 0 || layer >= a->L) return set_err(TG_E_INVALID, "layer %d out of range 0..%d", layer, a->L - 1);
    int rc = check_tokens(n_tokens);
    if (rc) return rc;
    if (!x || !moe_out) return set_err(TG_E_INVALID, "x / moe_out is NULL");
    const int dev = g_dev;
    if (dev < 0) return set_err(TG_E_NODEVICE, "no device initialised (tg_gpu_init)");
    if (dev >= NOALLOC_MAX_DEV) return set_err(TG_E_UNSUPPORTED, "device %d: no-alloc scratch covers devices 0..%d",
                                               dev, NOALLOC_MAX_DEV - 1);
    int cur = -1;
    HIP_TRY(hipGetDevice(&cur));
    if (cur != dev) HIP_TRY(hipSetDevice(dev));
    if (!g_na[dev].ptr && (rc = noalloc_setup(dev))) return rc;
    const int tmax = noalloc_tmax(a->s);
    if (n_tokens > tmax)
        return set_err(TG_E_INVALID,
                       "no-alloc layer call: %d tokens need %zu bytes of scratch, above its %zu (at most %d tokens at "
                       "this shape)",
                       n_tokens, scratch_layout(a->s, n_tokens, nullptr, nullptr),
                       NOALLOC_SCRATCH_BYTES - NOALLOC_HEADER, tmax);
    std::lock_guard<std::mutex> lk(g_na_mu);
    NoAllocDev &d = g_na[dev];
    Scratch c;
    scratch_layout(a->s, tmax, d.ptr + NOALLOC_HEADER, &c);
    c.dec_err = noalloc_err(d.ptr);  // one error word per device, whatever the layout
    hipStream_t st = as_stream(stream);
    // exchange words of another shape: back to zero (a kernel, not a memset node)
    HIP_TRY(tg::launch_keyed_clear(reinterpret_cast<uint64_t *>(d.ptr), noalloc_key(a->s),
                                   reinterpret_cast<uint32_t *>(c.dec), c.dec_bytes / 4, st));
    d.used = true;
    return moe_layer_launch(a, c, layer, x, moe_out, nullptr, n_tokens, topk_idx, topk_w, eps, st);
}

// Reads and clears one device-side error word (the first poll failure since
// it was last read).
static int take_err_word(uint32_t *word, uint32_t *v) {
    HIP_TRY(hipMemcpy(v, word, sizeof *v, hipMemcpyDeviceToHost));
    if (*v) {
        const uint32_t zero = 0u;
        HIP_TRY(hipMemcpy(word, &zero, sizeof zero, hipMemcpyHostToDevice));
    }
    return TG_OK;
}

extern "C" int tg_arena_status(tg_arena *a) {
    if (!a) return set_err(TG_E_INVALID, "arena is NULL");
    int rc = ensure_device();
    if (rc) return rc;
    HIP_TRY(hipDeviceSynchronize());
    uint32_t v = 0, vn = 0;
    if (a->sc.dec_err && (rc = take_err_word(a->sc.dec_err, &v))) return rc;
    if (g_dev >= 0 && g_dev < NOALLOC_MAX_DEV && g_na[g_dev].used &&  // the no-alloc call's error word
        (rc = take_err_word(noalloc_err(g_na[g_dev].ptr), &vn)))
        return rc;
    if (v) return set_err(TG_E_HIP, "MoE launch: a device-side wait ran out of tries (code %u)", v);
    if (vn) return set_err(TG_E_HIP, "no-alloc layer call: a device-side poll ran out of tries (code %u)", vn);
    return TG_OK;
}

extern "C" int tg_clock_mfma_mhz(int iters, double *mhz_median, double *mhz_min, double *mhz_max) {
    if (iters <= 0 || !mhz_median) return set_err(TG_E_INVALID, "tg_clock_mfma_mhz: iters %d, null output", iters);
    int rc = ensure_device();
    if (rc) return rc;
    int dev = 0, n_cu = 0;
    HIP_TRY(hipGetDevice(&dev));
    HIP_TRY(hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev));
    const int blocks = 4 * n_cu;
    unsigned long long *d = nullptr;
    if (hipMalloc(&d, sizeof(unsigned long long) * 4 * (size_t)blocks) != hipSuccess) {
        (void)hipGetLastError();
        return set_err(TG_E_NOMEM, "tg_clock_mfma_mhz: stamps");
    }
    std::vector<unsigned long long> h(4 * (size_t)blocks);
    hipError_t e = tg::launch_clock_mfma(d, blocks, iters, nullptr);
    if (e == hipSuccess) e = hipMemcpy(h.data(), d, sizeof(unsigned long long) * h.size(), hipMemcpyDeviceToHost);
    (void)hipFree(d);
    if (e != hipSuccess) return set_err(TG_E_HIP, "tg_clock_mfma_mhz: %s", hipGetErrorString(e));
    std::vector<double> mhz;
    for (int b = 0; b < blocks; b++) {
        const double cyc = (double)(h[4 * b + 2] - h[4 * b]), ticks = (double)(h[4 * b + 3] - h[4 * b + 1]);
        if (ticks > 0) mhz.push_back(cyc / (ticks / 100.0));  // 100 MHz real-time counter
    }
    if (mhz.empty()) return set_err(TG_E_HIP, "tg_clock_mfma_mhz: no elapsed real time");
    std::sort(mhz.begin(), mhz.end());
    *mhz_median = mhz[mhz.size() / 2];
    if (mhz_min) *mhz_min = mhz.front();
    if (mhz_max) *mhz_max = mhz.back();
    return TG_OK;
}

extern "C" int tg_debug_fault_inject(uint32_t spin_limit, int drop_line) {
    tg::set_fault_injection(spin_limit, drop_line);
    return TG_OK;
}

extern "C" int tg_moe_stack_q40(tg_arena *a, float *x, int n_tokens, int layer0, int n_layers, float eps) {
    int rc = stack_check(a, layer0, n_layers, n_tokens, x);
    if (rc) return rc;
    size_t nx = (size_t)n_tokens * a->s.H;
    HIP_TRY(hipMemcpy(a->xbuf, x, nx * sizeof(float), hipMemcpyHostToDevice));
    if ((rc = stack_run(a, a->xbuf, n_tokens, layer0, n_layers, eps, nullptr))) return rc;
    HIP_TRY(hipMemcpy(x, a->xbuf, nx * sizeof(float), hipMemcpyDeviceToHost));
    return tg_arena_status(a);
}

// ================================================================ building blocks
extern "C" int tg_q40_quantize_q8_0_dev(const float *x, void *q8_out, int n, void *stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!x || !q8_out || n <= 0 || n % 32) return set_err(TG_E_INVALID, "n must be a positive multiple of 32");
    HIP_TRY(tg::launch_quantize_q8_0(x, static_cast<uint8_t *>(q8_out), n, as_stream(stream)));
    return TG_OK;
}

extern "C" int tg_q40_to_planar_dev(const void *aos, void *planar, int rows, int nb, void *stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!aos || !planar || rows <= 0 || nb <= 0) return set_err(TG_E_INVALID, "bad repack arguments");
    HIP_TRY(tg::launch_repack_tensor(static_cast<const uint8_t *>(aos), static_cast<uint8_t *>(planar),
                                     (size_t)rows * nb, true, as_stream(stream)));
    return TG_OK;
}

extern "C" int tg_q40_from_planar_dev(const void *planar, void *aos, int rows, int nb, void *stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!aos || !planar || rows <= 0 || nb <= 0) return set_err(TG_E_INVALID, "bad repack arguments");
    HIP_TRY(tg::launch_repack_tensor(static_cast<const uint8_t *>(planar), static_cast<uint8_t *>(aos),
                                     (size_t)rows * nb, false, as_stream(stream)));
    return TG_OK;
}

extern "C" int tg_q40_block_sums_dev(const void *w_planar, int rows, int cols, const void *xq8, int32_t *sums,
                                     void *stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!w_planar || !xq8 || !sums || rows <= 0 || cols <= 0 || cols % 32)
        return set_err(TG_E_INVALID, "bad block-sum arguments");
    HIP_TRY(tg::launch_block_sums(static_cast<const uint8_t *>(w_planar), rows, cols / 32,
                                  static_cast<const uint8_t *>(xq8), sums, as_stream(stream)));
    return TG_OK;
}

extern "C" int tg_q40_matvec_dev(const void *w_planar, int rows, int cols, const void *xq8, float *out,
                                 void *stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!w_planar || !xq8 || !out || rows <= 0 || cols <= 0 || cols % 32 || cols / 32 > tg::MAX_NB)
        return set_err(TG_E_INVALID, "bad matvec arguments (cols multiple of 32, <= %d)", tg::MAX_NB * 32);
    HIP_TRY(tg::launch_matvec(static_cast<const uint8_t *>(w_planar), rows, cols / 32,
                              static_cast<const uint8_t *>(xq8), out, as_stream(stream)));
    return TG_OK;
}

extern "C" int tg_router_topk_dev(const float *Wr, const float *x, int n_experts, int embed_dim, int top_k,
                                  float eps, int n_tokens, float *logits, int32_t *topk_idx, float *topk_w,
                                  void *stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!Wr || !x || !logits) return set_err(TG_E_INVALID, "Wr / x / logits is NULL");
    if ((rc = check_shape(embed_dim, 32, n_experts, top_k))) return rc;
    if ((rc = check_tokens(n_tokens))) return rc;
    hipStream_t st = as_stream(stream);
    float *raw = nullptr;
    if (hipMalloc(&raw, sizeof(float) * (size_t)n_tokens * n_experts) != hipSuccess) {
        (void)hipGetLastError();
        return set_err(TG_E_NOMEM, "router scratch");
    }
    hipError_t e1 = tg::launch_route(Wr, x, n_tokens, n_experts, embed_dim, raw, st);
    hipError_t e2 = e1 == hipSuccess ? tg::launch_topk(raw, x, n_tokens, n_experts, embed_dim, top_k, eps, logits,
                                                       topk_idx, topk_w, st)
                                     : e1;
    hipError_t e3 = hipStreamSynchronize(st);
    dfree(raw);
    HIP_TRY(e2);
    HIP_TRY(e3);
    return TG_OK;
}

extern "C" int tg_stream_read_dev(const void *p, size_t nbytes, int grid, uint32_t *sink, void *stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!p || !sink || grid <= 0 || nbytes % 16) return set_err(TG_E_INVALID, "bad stream-read arguments");
    HIP_TRY(tg::launch_stream_read(p, nbytes, grid, sink, as_stream(stream)));
    return TG_OK;
}

extern "C" int tg_synth_normal_dev(uint64_t seed, uint64_t stream_id, float sigma, size_t n, float *out,
                                   void *stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!out) return set_err(TG_E_INVALID, "out is NULL");
    HIP_TRY(tg::launch_synth_normal(out, tg::host_stream_key(seed, stream_id), sigma, n, as_stream(stream)));
    return TG_OK;
}

extern "C" int tg_synth_q40_dev(uint64_t seed, uint64_t stream_id, float sigma, int rows, int cols,
                                void *planar_out, void *stream) {
    int rc = ensure_device();
    if (rc) return rc;
    if (!planar_out || rows <= 0 || cols <= 0 || cols % 32) return set_err(TG_E_INVALID, "bad synth arguments");
    HIP_TRY(tg::launch_synth_q40(static_cast<uint8_t *>(planar_out), tg::host_stream_key(seed, stream_id), sigma,
                                 rows, cols / 32, as_stream(stream)));
    return TG_OK;
}

// ================================================================ reference ABI
// Residency helpers: the same POSIX calls as csrc/libtinygiant.c:745-766
// (16 KiB page mask); with every expert resident in HBM they only matter
// for host buffers the caller still keeps.
static const uintptr_t kPageMask = ~((uintptr_t)16384 - 1);

extern "C" void tg_prefetch(const void *addr, size_t len) {
    void *aligned = (void *)((uintptr_t)addr & kPageMask);
    size_t alen = len + ((uintptr_t)addr - (uintptr_t)aligned);
    posix_madvise(aligned, alen, POSIX_MADV_WILLNEED);
}

extern "C" void tg_prefetch_batch(const void **addrs, const size_t *lens, int count) {
    for (int i = 0; i < count; i++) tg_prefetch(addrs[i], lens[i]);
}

static void mirror_add(const void *addr, size_t len);

// mlock of the 16 KiB-aligned range, as the reference; the range is also
// mirrored in HBM for the legacy entry points (residency section below).
extern "C" int tg_mlock(const void *addr, size_t len) {
    void *aligned = (void *)((uintptr_t)addr & kPageMask);
    size_t alen = len + ((uintptr_t)addr - (uintptr_t)aligned);
    const int rc = mlock(aligned, alen);
    mirror_add(addr, len);
    return rc;
}

// ================================================================ legacy ABI
// The reference's legacy entry points keep its conventions: synchronous
// calls on caller-owned host pointers, no error returns.  Q4_K / Q6_K / f16
// / f32 products, the RMS norm, the expert forward, attention decode and the
// transformer layer run on the GPU (tg_legacy.hip): each call copies its
// operands into one device scratch buffer (grown as needed, kept for the
// process), runs the kernels on one stream and copies the result back (and
// the new KV cache rows into the caller's caches).  A failure (no device,
// out of memory, an invalid geometry) is reported loudly: tg_last_error(),
// one line on stderr per symbol, and NaN in every output element.
static void legacy_fail(const char *name, std::atomic<bool> &warned) {
    if (!warned.exchange(true)) fprintf(stderr, "libtinygiant (gfx950): %s: %s\n", name, g_err.c_str());
}

static void fill_nan(float *p, long n) {
    if (!p) return;
    for (long i = 0; i < n; i++) p[i] = NAN;
}

#define LEGACY_FLAG(name) static std::atomic<bool> warned_##name{false}

LEGACY_FLAG(expert_forward);
LEGACY_FLAG(expert_forward_mixed);
LEGACY_FLAG(matmul_q4k);
LEGACY_FLAG(matmul_q6k);
LEGACY_FLAG(rms_norm);
LEGACY_FLAG(f32_matvec);
LEGACY_FLAG(f16_matvec);
LEGACY_FLAG(attention_decode);
LEGACY_FLAG(attention_decode_q4);
LEGACY_FLAG(transformer_layer);
LEGACY_FLAG(moe_forward);
LEGACY_FLAG(matmul_q4k_scalar);

// One device scratch buffer and stream for the legacy calls (one call at a
// time: the mutex serialises callers).
static std::mutex g_lg_mu;
static uint8_t *g_lg_buf = nullptr;
static size_t g_lg_cap = 0;
static int g_lg_dev = -1;
static hipStream_t g_lg_st = nullptr;

// Carves 256-byte aligned pieces of the scratch buffer; a first pass with no
// base only counts the bytes.
struct LgCarve {
    uint8_t *base;
    size_t off = 0;
    template <class T>
    T *take(size_t bytes) {
        const size_t o = (off + 255) & ~(size_t)255;
        off = o + bytes;
        return base ? reinterpret_cast<T *>(base + o) : nullptr;
    }
};

static size_t g_lg_pin_off = 0;  // bounce bytes handed out since the last wait (pinned buffer below)
static int lg_sync();

static int lg_reserve(size_t bytes) {
    int rc = ensure_device();
    if (rc) return rc;
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (g_lg_buf && g_lg_dev != dev) {  // scratch of another device
        HIP_TRY(hipSetDevice(g_lg_dev));
        (void)hipFree(g_lg_buf);
        if (g_lg_st) (void)hipStreamDestroy(g_lg_st);
        g_lg_buf = nullptr; g_lg_cap = 0; g_lg_st = nullptr;
        HIP_TRY(hipSetDevice(dev));
    }
    g_lg_dev = dev;
    if (!g_lg_st) HIP_TRY(hipStreamCreateWithFlags(&g_lg_st, hipStreamNonBlocking));
    if (g_lg_pin_off) {  // a call that failed before its closing wait left bounce slots taken
        int rc2 = lg_sync();
        if (rc2) return rc2;
    }
    if (bytes > g_lg_cap) {
        if (g_lg_buf) HIP_TRY(hipFree(g_lg_buf));
        g_lg_buf = nullptr;
        g_lg_cap = 0;
        const size_t want = (bytes + ((size_t)1 << 20) - 1) & ~(((size_t)1 << 20) - 1);
        if (hipMalloc(&g_lg_buf, want) != hipSuccess) {
            (void)hipGetLastError();
            g_lg_buf = nullptr;
            return set_err(TG_E_NOMEM, "legacy scratch of %zu bytes", want);
        }
        g_lg_cap = want;
    }
    return TG_OK;
}

// Copies of up to LG_PIN_MAX bytes go through a pinned bounce buffer (one
// DMA from pinned memory instead of the runtime's staging of pageable
// memory).  A call's bounce slots are handed out in order and reused only
// after the call's closing synchronisation; a call that fails before it
// leaves them taken until the next call that finishes, and copies that do
// not fit go straight from pageable memory.  Kept until process exit.
static uint8_t *g_lg_pin = nullptr;
constexpr size_t LG_PIN_BYTES = (size_t)1 << 20, LG_PIN_MAX = (size_t)256 << 10;

static void *lg_pin_take(size_t n) {
    if (n > LG_PIN_MAX) return nullptr;
    if (!g_lg_pin && hipHostMalloc(reinterpret_cast<void **>(&g_lg_pin), LG_PIN_BYTES, hipHostMallocDefault) !=
                         hipSuccess) {
        g_lg_pin = nullptr;
        return nullptr;
    }
    const size_t o = (g_lg_pin_off + 255) & ~(size_t)255;
    if (o + n > LG_PIN_BYTES) return nullptr;
    g_lg_pin_off = o + n;
    return g_lg_pin + o;
}

static int lg_h2d(void *dst, const void *src, size_t n) {
    if (!n) return TG_OK;
    if (void *p = lg_pin_take(n)) {
        memcpy(p, src, n);
        src = p;
    }
    HIP_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, g_lg_st));
    return TG_OK;
}

// Waits for the legacy stream; every bounce slot handed out before is free
// again afterwards.
static int lg_sync() {
    HIP_TRY(hipStreamSynchronize(g_lg_st));
    g_lg_pin_off = 0;  // every copy issued so far has completed
    return TG_OK;
}

static int lg_finish(void *host_dst, const void *dev_src, size_t n) {
    void *p = n ? lg_pin_take(n) : nullptr;
    if (n) HIP_TRY(hipMemcpyAsync(p ? p : host_dst, dev_src, n, hipMemcpyDeviceToHost, g_lg_st));
    int rc = lg_sync();
    if (rc) return rc;
    if (p) memcpy(host_dst, p, n);
    return TG_OK;
}

// ------------------------------------------------------------- residency
// The reference keeps its hot experts resident by locking their pages: the
// cache calls tg_mlock on each pinned expert's gate / up / down views, which
// are read-only mmap views of the relayout files (cache.py:31-67), and the
// engine locks every attention weight (engine.py:134-139).  Here tg_mlock
// also copies a range to HBM once, and every legacy entry point reads a
// weight operand that lies inside such a range from that copy instead of
// sending it over PCIe per call.
//
// Which ranges are copied (tg_mirror_mode): by default only ranges that lie
// wholly in mappings without write permission, such as the reference's
// expert views.  Their bytes cannot be changed through this process's
// mapping, so reading the copy gives what the reference's call reads.
// Writable memory (the engine's attention weights: numpy arrays) is copied
// only in mode TG_MIRROR_ALL, in which the caller promises that a locked
// range keeps its bytes until tg_mirror_drop.
//
// Every use of a copy first compares the range with what it held when
// locked: its first and last 64 bytes (hashed) and MIRROR_SAMPLES words
// spread evenly over it, each read only where it lies inside the operand the
// caller passed, so nothing outside [host, host + n) is read.  A mismatch
// (an address reused for other data, a buffer reloaded in place) drops the
// copy and the call reads host memory.  A rewrite that changes none of the
// sampled bytes is not seen: that is the promise of TG_MIRROR_ALL.  A copy is
// used only on the device it was made on.  All of it under g_lg_mu.
constexpr int MIRROR_SAMPLES = 16;
struct Mirror {
    size_t len;
    void *dev;
    int device;
    uint64_t head, tail;             // FNV-1a of the first / last min(64, len) bytes
    uint64_t word[MIRROR_SAMPLES];   // 8 bytes at mirror_sample_at(len, i)
};
static std::map<uintptr_t, Mirror> g_mirror;
static size_t g_mirror_bytes = 0;
static uint64_t g_mirror_hits = 0, g_mirror_misses = 0;
static int g_mirror_mode = -1;  // TG_MIRROR_*; -1: from TG_MLOCK_MIRROR at first use

static uint64_t fnv(const uint8_t *b, size_t n) {
    uint64_t h = 1469598103934665603ull ^ n;
    for (size_t i = 0; i < n; i++) h = (h ^ b[i]) * 1099511628211ull;
    return h;
}

static size_t mirror_sample_at(size_t len, int i) {
    return len < 8 ? 0 : (len - 8) / (MIRROR_SAMPLES - 1) * (size_t)i;
}

static uint64_t load8(const uint8_t *p) {
    uint64_t v;
    memcpy(&v, p, 8);
    return v;
}

static int mirror_mode() {
    if (g_mirror_mode < 0) {
        const char *e = getenv("TG_MLOCK_MIRROR");
        g_mirror_mode = !e ? TG_MIRROR_READONLY
                        : e[0] == '0' ? TG_MIRROR_OFF
                        : strcmp(e, "all") == 0 ? TG_MIRROR_ALL
                                                : TG_MIRROR_READONLY;
    }
    return g_mirror_mode;
}

// Whether every page of [addr, addr + len) lies in a mapping of this process
// without write permission (/proc/self/maps).
static bool range_readonly(const void *addr, size_t len) {
    FILE *f = fopen("/proc/self/maps", "r");
    if (!f) return false;
    uintptr_t cur = (uintptr_t)addr;
    const uintptr_t end = cur + len;
    char line[512];
    while (cur < end && fgets(line, sizeof line, f)) {
        unsigned long lo = 0, hi = 0;
        char perm[8] = {0};
        if (sscanf(line, "%lx-%lx %7s", &lo, &hi, perm) != 3) continue;
        if (cur >= lo && cur < hi) {
            if (perm[1] == 'w') break;
            cur = hi;
        }
    }
    fclose(f);
    return cur >= end;
}

static void mirror_erase(std::map<uintptr_t, Mirror>::iterator it) {
    (void)hipFree(it->second.dev);
    g_mirror_bytes -= it->second.len;
    g_mirror.erase(it);
}

// Whether the locked range starting at a still holds its bytes, judged from
// the parts of it that lie in the caller's window [w0, w1).
static bool mirror_intact(uintptr_t a, const Mirror &m, uintptr_t w0, uintptr_t w1) {
    const size_t e = m.len < 64 ? m.len : 64;
    if (w0 == a && w1 - w0 >= e && fnv(reinterpret_cast<const uint8_t *>(a), e) != m.head) return false;
    if (w1 == a + m.len && w1 - w0 >= e && fnv(reinterpret_cast<const uint8_t *>(w1 - e), e) != m.tail) return false;
    if (m.len < 8) return true;
    for (int i = 0; i < MIRROR_SAMPLES; i++) {
        const uintptr_t p = a + mirror_sample_at(m.len, i);
        if (p >= w0 && p + 8 <= w1 && load8(reinterpret_cast<const uint8_t *>(p)) != m.word[i]) return false;
    }
    return true;
}

// The device copy of [host, host + n), or NULL.
static const void *mirror_find(const void *host, size_t n) {
    if (g_mirror.empty() || !host) return nullptr;
    auto it = g_mirror.upper_bound((uintptr_t)host);
    if (it == g_mirror.begin()) return nullptr;
    --it;
    const uintptr_t a = it->first, w0 = (uintptr_t)host, w1 = w0 + n;
    const Mirror &m = it->second;
    if (w1 > a + m.len || m.device != g_lg_dev) return nullptr;
    if (!mirror_intact(a, m, w0, w1)) {  // the range holds other bytes now
        mirror_erase(it);
        return nullptr;
    }
    return static_cast<const uint8_t *>(m.dev) + (w0 - a);
}

static void mirror_add(const void *addr, size_t len) {
    if (!addr || !len) return;
    std::lock_guard<std::mutex> lk(g_lg_mu);
    const int mode = mirror_mode();
    if (mode == TG_MIRROR_OFF || (mode == TG_MIRROR_READONLY && !range_readonly(addr, len))) return;
    const std::string err = g_err;  // best effort: the caller sees mlock's result only
    if (lg_reserve(0) == TG_OK) {
        auto it = g_mirror.find((uintptr_t)addr);
        if (it != g_mirror.end() && it->second.len >= len && it->second.device == g_lg_dev &&
            mirror_intact(it->first, it->second, (uintptr_t)addr, (uintptr_t)addr + it->second.len)) {
            g_err = err;
            return;  // already copied
        }
        void *d = nullptr;
        if (hipMalloc(&d, len) == hipSuccess) {
            if (hipMemcpy(d, addr, len, hipMemcpyHostToDevice) == hipSuccess) {
                if (it != g_mirror.end()) mirror_erase(it);  // an older copy of the same start
                const uint8_t *b = static_cast<const uint8_t *>(addr);
                const size_t e = len < 64 ? len : 64;
                Mirror m{len, d, g_lg_dev, fnv(b, e), fnv(b + len - e, e), {}};
                if (len >= 8)
                    for (int i = 0; i < MIRROR_SAMPLES; i++) m.word[i] = load8(b + mirror_sample_at(len, i));
                g_mirror[(uintptr_t)addr] = m;
                g_mirror_bytes += len;
            } else {
                (void)hipFree(d);
            }
        }
        (void)hipGetLastError();
    }
    g_err = err;
}

extern "C" int tg_mirror_mode(int mode) {
    std::lock_guard<std::mutex> lk(g_lg_mu);
    if (mode < 0) return mirror_mode();
    if (mode != TG_MIRROR_OFF && mode != TG_MIRROR_READONLY && mode != TG_MIRROR_ALL)
        return set_err(TG_E_INVALID, "tg_mirror_mode: unknown mode %d", mode);
    g_mirror_mode = mode;
    return mode;
}

extern "C" void tg_mirror_drop(const void *addr, size_t len) {
    std::lock_guard<std::mutex> lk(g_lg_mu);
    const uintptr_t lo = (uintptr_t)addr, hi = lo + len;
    for (auto it = g_mirror.begin(); it != g_mirror.end();) {
        auto nx = std::next(it);
        if (!addr || (it->first < hi && it->first + it->second.len > lo)) mirror_erase(it);
        it = nx;
    }
}

extern "C" void tg_mirror_stats(size_t *bytes, int *ranges, uint64_t *hits, uint64_t *misses) {
    std::lock_guard<std::mutex> lk(g_lg_mu);
    if (bytes) *bytes = g_mirror_bytes;
    if (ranges) *ranges = (int)g_mirror.size();
    if (hits) *hits = g_mirror_hits;
    if (misses) *misses = g_mirror_misses;
}

// A read-only operand of a legacy call: its HBM copy when tg_mlock made one,
// else copied into dst.
template <class T>
static int lg_in(const void *host, size_t n, T *dst, const T **out) {
    if (const void *m = mirror_find(host, n)) {
        g_mirror_hits++;
        *out = static_cast<const T *>(m);
        return TG_OK;
    }
    g_mirror_misses++;
    *out = dst;
    return lg_h2d(dst, host, n);
}

static size_t down_bytes(int fmt, int embed, int inter) {
    if (fmt == 1) return (size_t)embed * inter * 2;
    if (fmt == 2) return (size_t)embed * (inter / tg::LG_QK) * tg::LG_Q6K_BYTES;
    return (size_t)embed * (inter / tg::LG_QK) * tg::LG_Q4K_BYTES;
}

// Device buffers of one expert forward (activations only).
struct LgExpertBufs {
    void *xq, *hq;
    float *g, *u, *h, *dn;
};

static LgExpertBufs lg_expert_bufs(LgCarve &c, int embed, int inter) {
    LgExpertBufs b;
    b.xq = c.take<uint8_t>((size_t)(embed / tg::LG_QK) * tg::LG_Q8K_BYTES);
    b.hq = c.take<uint8_t>((size_t)(inter / tg::LG_QK) * tg::LG_Q8K_BYTES);
    b.g = c.take<float>(8 * (size_t)inter);  // gate rows, then the up rows (one expert's gate | up)
    b.u = b.g + inter;
    b.h = c.take<float>(4 * (size_t)inter);
    b.dn = c.take<float>(4 * (size_t)embed);
    return b;
}

// tg_moe_forward with every expert staged first, then the whole block in
// three launches (the Q8 of x and gate / up of every expert, SiLU and Q8 of
// every h, the down rows summed over the experts in order): the same bytes as
// the expert-by-expert chain (TG_LEGACY_MOE_ALL=0 keeps that chain, here
// and for a single expert with a Q4_K down matrix).
static bool lg_moe_all_enabled() {
    static const bool on = [] {
        const char *v = getenv("TG_LEGACY_MOE_ALL");
        return !(v && v[0] == '0');
    }();
    return on;
}

// expert_forward_mixed on device operands (libtinygiant.c:599-643):
// Q8(x), gate and up rows, SiLU(gate) * up, down by format (1 f16, 2 Q6_K,
// otherwise Q4_K), out += weight * down.
static int lg_expert(const uint8_t *gate, const uint8_t *up, const void *down, int fmt, const float *x, float *out,
                     float weight, int embed, int inter, const LgExpertBufs &b) {
    const int gbpr = embed / tg::LG_QK, dbpr = inter / tg::LG_QK;
    hipStream_t st = g_lg_st;
    if (fmt == 0 && tg::moe_q4k_ok(1, embed, inter) && lg_moe_all_enabled()) {
        // Q4_K down: the fused launches for one expert (Q8 of x and gate | up,
        // SiLU + Q8, down added to out as out + weight * down)
        tg::LgMoeOps P{};
        P.gate[0] = gate;
        P.up[0] = up;
        P.down[0] = static_cast<const uint8_t *>(down);
        P.w[0] = weight;
        PROFILED("lg_moe_gateup", st, tg::launch_moe_gateup_q4k(P, 1, x, b.g, embed, inter, st));
        PROFILED("lg_moe_silu", st, tg::launch_moe_silu_q8k(b.g, b.hq, 1, inter, st));
        PROFILED("lg_moe_down", st, tg::launch_moe_down_acc_q4k(P, 1, b.hq, out, embed, inter, true, st));
        return TG_OK;
    }
    PROFILED("lg_quant", st, tg::launch_quantize_q8k(x, b.xq, gbpr, st));
    PROFILED("lg_q4k", st, tg::launch_matmul_q4k(gate, b.xq, b.g, inter, gbpr, st));
    PROFILED("lg_q4k", st, tg::launch_matmul_q4k(up, b.xq, b.u, inter, gbpr, st));
    PROFILED("lg_silu", st, tg::launch_silu_mul_vec(b.g, b.u, b.h, inter, st));
    if (fmt == 1) {
        PROFILED("lg_f16", st, tg::launch_matvec_two_acc(down, true, b.h, b.dn, embed, inter, st));
    } else {
        PROFILED("lg_quant", st, tg::launch_quantize_q8k(b.h, b.hq, dbpr, st));
        if (fmt == 2)
            PROFILED("lg_q6k", st,
                     tg::launch_matmul_q6k(static_cast<const uint8_t *>(down), b.hq, b.dn, embed, dbpr, st));
        else
            PROFILED("lg_q4k_down", st,
                     tg::launch_matmul_q4k(static_cast<const uint8_t *>(down), b.hq, b.dn, embed, dbpr, st));
    }
    PROFILED("lg_acc", st, tg::launch_acc_scaled(out, b.dn, weight, embed, st));
    return TG_OK;
}

static int lg_expert_forward_mixed(const uint8_t *gate, const uint8_t *up, const void *down, int fmt,
                                   const float *input, float *output, float weight, int embed, int inter) {
    const int gbpr = embed / tg::LG_QK;
    const size_t gb = (size_t)inter * gbpr * tg::LG_Q4K_BYTES, db = down_bytes(fmt, embed, inter);
    for (int pass = 0; pass < 2; pass++) {
        LgCarve c{pass ? g_lg_buf : nullptr};
        uint8_t *dg = c.take<uint8_t>(gb), *du = c.take<uint8_t>(gb), *dd = c.take<uint8_t>(db);
        float *dx = c.take<float>(4 * (size_t)embed), *dout = c.take<float>(4 * (size_t)embed);
        const LgExpertBufs b = lg_expert_bufs(c, embed, inter);
        if (!pass) {
            int rc = lg_reserve(c.off);
            if (rc) return rc;
            continue;
        }
        int rc;
        const uint8_t *pg, *pu, *pd;
        if ((rc = lg_in(gate, gb, dg, &pg)) || (rc = lg_in(up, gb, du, &pu)) || (rc = lg_in(down, db, dd, &pd)) ||
            (rc = lg_h2d(dx, input, 4 * (size_t)embed)) || (rc = lg_h2d(dout, output, 4 * (size_t)embed)) ||
            (rc = lg_expert(pg, pu, pd, fmt, dx, dout, weight, embed, inter, b)))
            return rc;
        return lg_finish(output, dout, 4 * (size_t)embed);
    }
    return TG_OK;
}

extern "C" void tg_expert_forward(const uint8_t *q4_data, const float *input, float *output, float weight,
                                  int embed_dim, int inter_dim) {
    if (embed_dim <= 0 || inter_dim <= 0) return;
    std::lock_guard<std::mutex> lk(g_lg_mu);
    const size_t gb = (size_t)inter_dim * (embed_dim / tg::LG_QK) * tg::LG_Q4K_BYTES;
    if (lg_expert_forward_mixed(q4_data, q4_data + gb, q4_data + 2 * gb, 0, input, output, weight, embed_dim,
                                inter_dim)) {
        legacy_fail("tg_expert_forward", warned_expert_forward);
        fill_nan(output, embed_dim);
    }
}

extern "C" void tg_expert_forward_mixed(const uint8_t *gate_q4, const uint8_t *up_q4, const void *down_data,
                                        int down_format, const float *input, float *output, float weight,
                                        int embed_dim, int inter_dim) {
    if (embed_dim <= 0 || inter_dim <= 0) return;
    std::lock_guard<std::mutex> lk(g_lg_mu);
    if (lg_expert_forward_mixed(gate_q4, up_q4, down_data, down_format, input, output, weight, embed_dim,
                                inter_dim)) {
        legacy_fail("tg_expert_forward_mixed", warned_expert_forward_mixed);
        fill_nan(output, embed_dim);
    }
}


// after the chain's buffers: every expert's staging (for experts not held in
// HBM), the gate / up rows of all experts and their Q8 h blocks
struct LgMoeAllBufs {
    uint8_t *stage;
    float *gu;
    void *hq;
};
static LgMoeAllBufs lg_moe_all_carve(LgCarve &c, int n_exp, int embed, int inter, size_t eb) {
    LgMoeAllBufs m;
    m.stage = c.take<uint8_t>((size_t)n_exp * eb);
    m.gu = c.take<float>(4 * (size_t)n_exp * 2 * inter);
    m.hq = c.take<uint8_t>((size_t)n_exp * (inter / tg::LG_QK) * tg::LG_Q8K_BYTES);
    (void)embed;
    return m;
}

// each expert's gate, up and down (Q4_K) from its HBM copy or staged
static int lg_moe_ops(int n, const uint8_t *const *gp, const uint8_t *const *up, const void *const *dp,
                      const float *w, size_t gb, size_t db, uint8_t *stage, tg::LgMoeOps &P) {
    P = tg::LgMoeOps{};
    for (int e = 0; e < n; e++) {
        uint8_t *de = stage + (size_t)e * (2 * gb + db);
        int rc;
        if ((rc = lg_in(gp[e], gb, de, &P.gate[e])) || (rc = lg_in(up[e], gb, de + gb, &P.up[e])) ||
            (rc = lg_in(static_cast<const uint8_t *>(dp[e]), db, de + 2 * gb, &P.down[e])))
            return rc;
        P.w[e] = w[e];
    }
    return TG_OK;
}

// out = sum over the experts in order of weight * down(SiLU(gate x) * up x),
// x the device input (its Q8 blocks formed inside the gate / up launch)
static int lg_moe_run(const tg::LgMoeOps &P, int n, const float *x, float *out, int embed, int inter,
                      const LgExpertBufs &b, const LgMoeAllBufs &m) {
    hipStream_t st = g_lg_st;
    PROFILED("lg_moe_gateup", st, tg::launch_moe_gateup_q4k(P, n, x, m.gu, embed, inter, st));
    PROFILED("lg_moe_silu", st, tg::launch_moe_silu_q8k(m.gu, m.hq, n, inter, st));
    PROFILED("lg_moe_down", st, tg::launch_moe_down_acc_q4k(P, n, m.hq, out, embed, inter, false, st));
    return TG_OK;
}

static int lg_moe_all(const uint8_t **expert_ptrs, const float *weights, int n_experts, const float *dx, float *dout,
                      float *output, int embed, int inter, size_t gb, size_t eb, const LgExpertBufs &b, LgCarve &c) {
    const LgMoeAllBufs m = lg_moe_all_carve(c, n_experts, embed, inter, eb);
    const uint8_t *gp[tg::LG_MOE_MAX], *up[tg::LG_MOE_MAX];
    const void *dp[tg::LG_MOE_MAX];
    for (int e = 0; e < n_experts; e++) {  // gate, up and down one after another in each expert's bytes
        gp[e] = expert_ptrs[e];
        up[e] = expert_ptrs[e] + gb;
        dp[e] = expert_ptrs[e] + 2 * gb;
    }
    tg::LgMoeOps P;
    int rc;
    if ((rc = lg_moe_ops(n_experts, gp, up, dp, weights, gb, eb - 2 * gb, m.stage, P)) ||
        (rc = lg_moe_run(P, n_experts, dx, dout, embed, inter, b, m)))
        return rc;
    return lg_finish(output, dout, 4 * (size_t)embed);
}

extern "C" void tg_moe_forward(const uint8_t **expert_ptrs, const float *weights, int n_experts, const float *input,
                               float *output, int embed_dim, int inter_dim) {
    if (embed_dim <= 0 || inter_dim <= 0) return;
    std::lock_guard<std::mutex> lk(g_lg_mu);
    const size_t gb = (size_t)inter_dim * (embed_dim / tg::LG_QK) * tg::LG_Q4K_BYTES;
    const size_t eb = 2 * gb + down_bytes(0, embed_dim, inter_dim);
    const bool moe_all = tg::moe_q4k_ok(n_experts, embed_dim, inter_dim) && lg_moe_all_enabled();
    auto run = [&]() -> int {
        for (int pass = 0; pass < 2; pass++) {
            LgCarve c{pass ? g_lg_buf : nullptr};
            uint8_t *de = c.take<uint8_t>(moe_all ? 0 : eb);
            float *dx = c.take<float>(4 * (size_t)embed_dim), *dout = c.take<float>(4 * (size_t)embed_dim);
            const LgExpertBufs b = lg_expert_bufs(c, embed_dim, inter_dim);
            if (!pass) {
                if (moe_all) lg_moe_all_carve(c, n_experts, embed_dim, inter_dim, eb);
                int rc = lg_reserve(c.off);
                if (rc) return rc;
                continue;
            }
            int rc = lg_h2d(dx, input, 4 * (size_t)embed_dim);
            if (rc) return rc;
            if (moe_all) {  // every expert in three launches; the down launch writes every output row
                return lg_moe_all(expert_ptrs, weights, n_experts, dx, dout, output, embed_dim, inter_dim, gb, eb,
                                  b, c);
            }
            HIP_TRY(hipMemsetAsync(dout, 0, 4 * (size_t)embed_dim, g_lg_st));  // the reference's memset
            for (int e = 0; e < n_experts; e++) {
                // one expert's bytes at a time: a copy waits for the previous expert's kernels
                const uint8_t *pg, *pu, *pd, *src = expert_ptrs[e];
                if ((rc = lg_in(src, gb, de, &pg)) || (rc = lg_in(src + gb, gb, de + gb, &pu)) ||
                    (rc = lg_in(src + 2 * gb, eb - 2 * gb, de + 2 * gb, &pd)) ||
                    (rc = lg_expert(pg, pu, pd, 0, dx, dout, weights[e], embed_dim, inter_dim, b)))
                    return rc;
            }
            return lg_finish(output, dout, 4 * (size_t)embed_dim);
        }
        return TG_OK;
    };
    if (run()) {
        legacy_fail("tg_moe_forward", warned_moe_forward);
        fill_nan(output, embed_dim);
    }
}

// nrows x (ncols / 256) blocks of Q4_K or Q6_K times the input's Q8 blocks
static int lg_matmul_k(bool q6, const uint8_t *W, const float *input, float *output, int nrows, int ncols,
                       bool scalar) {
    const int bpr = ncols / tg::LG_QK;
    const size_t wb = (size_t)nrows * bpr * (q6 ? tg::LG_Q6K_BYTES : tg::LG_Q4K_BYTES);
    const size_t xb = 4 * (size_t)bpr * tg::LG_QK;
    for (int pass = 0; pass < 2; pass++) {
        LgCarve c{pass ? g_lg_buf : nullptr};
        uint8_t *dw = c.take<uint8_t>(wb);
        float *dx = c.take<float>(xb);
        void *dq = c.take<uint8_t>((size_t)bpr * tg::LG_Q8K_BYTES);
        float *dy = c.take<float>(4 * (size_t)nrows);
        if (!pass) {
            int rc = lg_reserve(c.off);
            if (rc) return rc;
            continue;
        }
        int rc;
        const uint8_t *pw;
        if ((rc = lg_in(W, wb, dw, &pw)) || (rc = lg_h2d(dx, input, xb))) return rc;
        if (scalar) {
            HIP_TRY(tg::launch_matmul_q4k_scalar(pw, dx, dy, nrows, bpr, g_lg_st));
        } else {
            HIP_TRY(tg::launch_quantize_q8k(dx, dq, bpr, g_lg_st));
            if (q6)
                HIP_TRY(tg::launch_matmul_q6k(pw, dq, dy, nrows, bpr, g_lg_st));
            else
                HIP_TRY(tg::launch_matmul_q4k(pw, dq, dy, nrows, bpr, g_lg_st));
        }
        return lg_finish(output, dy, 4 * (size_t)nrows);
    }
    return TG_OK;
}

extern "C" void tg_matmul_q4k(const uint8_t *q4_matrix, const float *input, float *output, int nrows, int ncols) {
    if (nrows <= 0) return;
    std::lock_guard<std::mutex> lk(g_lg_mu);
    if (lg_matmul_k(false, q4_matrix, input, output, nrows, ncols, false)) {
        legacy_fail("tg_matmul_q4k", warned_matmul_q4k);
        fill_nan(output, nrows);
    }
}

extern "C" void tg_matmul_q6k(const uint8_t *q6_matrix, const float *input, float *output, int nrows, int ncols) {
    if (nrows <= 0) return;
    std::lock_guard<std::mutex> lk(g_lg_mu);
    if (lg_matmul_k(true, q6_matrix, input, output, nrows, ncols, false)) {
        legacy_fail("tg_matmul_q6k", warned_matmul_q6k);
        fill_nan(output, nrows);
    }
}

extern "C" void tg_matmul_q4k_scalar(const uint8_t *q4_matrix, const float *input, float *output, int nrows,
                                     int ncols) {
    if (nrows <= 0) return;
    std::lock_guard<std::mutex> lk(g_lg_mu);
    if (lg_matmul_k(false, q4_matrix, input, output, nrows, ncols, true)) {
        legacy_fail("tg_matmul_q4k_scalar", warned_matmul_q4k_scalar);
        fill_nan(output, nrows);
    }
}

// f16 (half) or f32 matrix nrows x ncols times x
static int lg_matvec(bool half, const void *A, const float *x, float *out, int nrows, int ncols) {
    const size_t ab = (size_t)nrows * ncols * (half ? 2 : 4);
    for (int pass = 0; pass < 2; pass++) {
        LgCarve c{pass ? g_lg_buf : nullptr};
        uint8_t *da = c.take<uint8_t>(ab);
        float *dx = c.take<float>(4 * (size_t)ncols), *dy = c.take<float>(4 * (size_t)nrows);
        if (!pass) {
            int rc = lg_reserve(c.off);
            if (rc) return rc;
            continue;
        }
        int rc;
        const uint8_t *pa;
        if ((rc = lg_in(A, ab, da, &pa)) || (rc = lg_h2d(dx, x, 4 * (size_t)ncols))) return rc;
        HIP_TRY(tg::launch_matvec_two_acc(pa, half, dx, dy, nrows, ncols, g_lg_st));
        return lg_finish(out, dy, 4 * (size_t)nrows);
    }
    return TG_OK;
}

extern "C" void tg_f32_matvec(const float *A, const float *x, float *out, int nrows, int ncols) {
    if (nrows <= 0 || ncols < 0) return;
    std::lock_guard<std::mutex> lk(g_lg_mu);
    if (lg_matvec(false, A, x, out, nrows, ncols)) {
        legacy_fail("tg_f32_matvec", warned_f32_matvec);
        fill_nan(out, nrows);
    }
}

extern "C" void tg_f16_matvec(const uint16_t *A, const float *x, float *out, int nrows, int ncols) {
    if (nrows <= 0 || ncols < 0) return;
    std::lock_guard<std::mutex> lk(g_lg_mu);
    if (lg_matvec(true, A, x, out, nrows, ncols)) {
        legacy_fail("tg_f16_matvec", warned_f16_matvec);
        fill_nan(out, nrows);
    }
}

extern "C" void tg_rms_norm(const float *x, const float *weight, float *out, int dim, float eps) {
    if (dim <= 0) return;
    std::lock_guard<std::mutex> lk(g_lg_mu);
    auto run = [&]() -> int {
        for (int pass = 0; pass < 2; pass++) {
            LgCarve c{pass ? g_lg_buf : nullptr};
            float *dx = c.take<float>(4 * (size_t)dim), *dw = c.take<float>(4 * (size_t)dim);
            float *dy = c.take<float>(4 * (size_t)dim);
            if (!pass) {
                int rc = lg_reserve(c.off);
                if (rc) return rc;
                continue;
            }
            int rc;
            if ((rc = lg_h2d(dx, x, 4 * (size_t)dim)) || (rc = lg_h2d(dw, weight, 4 * (size_t)dim))) return rc;
            HIP_TRY(tg::launch_rms_norm(dx, dw, dy, dim, eps, g_lg_st));
            return lg_finish(out, dy, 4 * (size_t)dim);
        }
        return TG_OK;
    };
    if (run()) {
        legacy_fail("tg_rms_norm", warned_rms_norm);
        fill_nan(out, dim);
    }
}

// ---------------------------------------------------------------- attention
// Geometry of one attention decode step (libtinygiant.c:365-551).
struct LgAttn {
    int embed, n_heads, n_kv, hd, kv_len, kv_max, pos;
    int q_dim() const { return n_heads * hd; }
    int kv_dim() const { return n_kv * hd; }
    int seq() const { return kv_len + 1; }
    bool ok() const {
        return embed > 0 && n_heads > 0 && n_kv > 0 && n_heads % n_kv == 0 && hd > 0 && hd % 2 == 0 && hd <= 512 &&
               kv_len >= 0 && kv_len < kv_max && pos >= 0;
    }
};

// Device buffers of one attention step (weights excluded).
struct LgAttnBufs {
    float *x, *q, *k, *v, *qn, *kn, *ao, *out, *kc, *vc, *scr, *cs, *sn;
    void *xq, *aq;
};

static LgAttnBufs lg_attn_bufs(LgCarve &c, const LgAttn &g) {
    LgAttnBufs b;
    const size_t cache = 4 * (size_t)g.n_kv * g.seq() * g.hd;
    b.x = c.take<float>(4 * (size_t)g.embed);
    b.q = c.take<float>(4 * (size_t)g.q_dim());
    b.k = c.take<float>(4 * (size_t)g.kv_dim());
    b.v = c.take<float>(4 * (size_t)g.kv_dim());
    b.qn = c.take<float>(4 * (size_t)g.q_dim());
    b.kn = c.take<float>(4 * (size_t)g.kv_dim());
    b.ao = c.take<float>(4 * (size_t)g.q_dim());
    b.out = c.take<float>(4 * (size_t)g.embed);
    b.kc = c.take<float>(cache);
    b.vc = c.take<float>(cache);
    b.scr = c.take<float>(sizeof(float) * tg::attn_scratch_floats(g.n_heads, g.seq()));
    b.cs = c.take<float>(4 * (size_t)(g.hd / 2));
    b.sn = c.take<float>(4 * (size_t)(g.hd / 2));
    b.xq = c.take<uint8_t>((size_t)(g.embed / tg::LG_QK) * tg::LG_Q8K_BYTES);
    b.aq = c.take<uint8_t>((size_t)(g.q_dim() / tg::LG_QK) * tg::LG_Q8K_BYTES);
    return b;
}

// Host cache rows 0 .. kv_len-1 of every kv head into the device caches
// [n_kv][seq][hd], and this position's RoPE table rows.
static int lg_attn_in(const LgAttn &g, const LgAttnBufs &b, const float *kv_k, const float *kv_v,
                      const float *rope_cos, const float *rope_sin) {
    const size_t row = 4 * (size_t)g.hd, half = 4 * (size_t)(g.hd / 2);
    if (g.kv_len > 0) {
        HIP_TRY(hipMemcpy2DAsync(b.kc, row * g.seq(), kv_k, row * g.kv_max, row * g.kv_len, g.n_kv,
                                 hipMemcpyHostToDevice, g_lg_st));
        HIP_TRY(hipMemcpy2DAsync(b.vc, row * g.seq(), kv_v, row * g.kv_max, row * g.kv_len, g.n_kv,
                                 hipMemcpyHostToDevice, g_lg_st));
    }
    int rc;
    if ((rc = lg_h2d(b.cs, rope_cos + (size_t)g.pos * (g.hd / 2), half)) ||
        (rc = lg_h2d(b.sn, rope_sin + (size_t)g.pos * (g.hd / 2), half)))
        return rc;
    return TG_OK;
}

// The new cache rows (row kv_len of every kv head) back to the host caches.
static int lg_attn_out(const LgAttn &g, const LgAttnBufs &b, float *kv_k, float *kv_v) {
    const size_t row = 4 * (size_t)g.hd;
    HIP_TRY(hipMemcpy2DAsync(kv_k + (size_t)g.kv_len * g.hd, row * g.kv_max, b.kc + (size_t)g.kv_len * g.hd,
                             row * g.seq(), row, g.n_kv, hipMemcpyDeviceToHost, g_lg_st));
    HIP_TRY(hipMemcpy2DAsync(kv_v + (size_t)g.kv_len * g.hd, row * g.kv_max, b.vc + (size_t)g.kv_len * g.hd,
                             row * g.seq(), row, g.n_kv, hipMemcpyDeviceToHost, g_lg_st));
    return TG_OK;
}

// The attention step on device operands (input b.x, output b.out): q/k/v
// projections (q4: Q4_K q, k, o and f16 v; else f32), per-head RMS norms of
// q and k (eps 1e-6), RoPE, the new rows into the caches, GQA attention,
// output projection.
static int lg_attn_core(bool q4, const void *wq, const void *wk, const void *wv, const void *wo, const float *qnw,
                        const float *knw, const LgAttn &g, const LgAttnBufs &b) {
    hipStream_t st = g_lg_st;
    const int ebpr = g.embed / tg::LG_QK;
    if (q4) {
        PROFILED("lg_quant", st, tg::launch_quantize_q8k(b.x, b.xq, ebpr, st));
        PROFILED("lg_q4k_attn", st,
                 tg::launch_matmul_q4k(static_cast<const uint8_t *>(wq), b.xq, b.q, g.q_dim(), ebpr, st));
        PROFILED("lg_q4k_attn", st,
                 tg::launch_matmul_q4k(static_cast<const uint8_t *>(wk), b.xq, b.k, g.kv_dim(), ebpr, st));
        PROFILED("lg_f16", st, tg::launch_matvec_two_acc(wv, true, b.x, b.v, g.kv_dim(), g.embed, st));
    } else {
        PROFILED("lg_f32", st, tg::launch_matvec_two_acc(wq, false, b.x, b.q, g.q_dim(), g.embed, st));
        PROFILED("lg_f32", st, tg::launch_matvec_two_acc(wk, false, b.x, b.k, g.kv_dim(), g.embed, st));
        PROFILED("lg_f32", st, tg::launch_matvec_two_acc(wv, false, b.x, b.v, g.kv_dim(), g.embed, st));
    }
    PROFILED("lg_rms", st, tg::launch_rms_norm_rows(b.q, qnw, b.qn, g.hd, g.n_heads, 1e-6f, st));
    PROFILED("lg_rms", st, tg::launch_rms_norm_rows(b.k, knw, b.kn, g.hd, g.n_kv, 1e-6f, st));
    PROFILED("lg_rope", st, tg::launch_rope(b.qn, g.n_heads, g.hd, b.cs, b.sn, st));
    PROFILED("lg_rope", st, tg::launch_rope(b.kn, g.n_kv, g.hd, b.cs, b.sn, st));
    PROFILED("lg_kv", st, tg::launch_kv_append(b.kn, b.v, b.kc, b.vc, g.n_kv, g.seq(), g.hd, g.kv_len, st));
    const float inv_sqrt = 1.0f / sqrtf((float)g.hd);
    PROFILED("lg_attn_sc", st,
             tg::launch_attn_scores(b.qn, b.kc, b.scr, g.n_heads, g.seq(), g.hd, g.n_heads / g.n_kv, inv_sqrt, st));
    PROFILED("lg_attn_sm", st, tg::launch_attn_softmax(b.scr, g.n_heads, g.seq(), st));
    PROFILED("lg_attn", st, tg::launch_attn_wv(b.scr, b.vc, b.ao, g.n_heads, g.seq(), g.hd, g.n_heads / g.n_kv, st));
    if (q4) {
        const int abpr = g.q_dim() / tg::LG_QK;
        PROFILED("lg_quant", st, tg::launch_quantize_q8k(b.ao, b.aq, abpr, st));
        PROFILED("lg_q4k_attn", st,
                 tg::launch_matmul_q4k(static_cast<const uint8_t *>(wo), b.aq, b.out, g.embed, abpr, st));
    } else {
        PROFILED("lg_f32", st, tg::launch_matvec_two_acc(wo, false, b.ao, b.out, g.embed, g.q_dim(), st));
    }
    return TG_OK;
}

// Bytes of the four projection weights.
static void lg_attn_wbytes(bool q4, const LgAttn &g, size_t &bq, size_t &bk, size_t &bv, size_t &bo) {
    if (q4) {
        bq = (size_t)g.q_dim() * (g.embed / tg::LG_QK) * tg::LG_Q4K_BYTES;
        bk = (size_t)g.kv_dim() * (g.embed / tg::LG_QK) * tg::LG_Q4K_BYTES;
        bv = (size_t)g.kv_dim() * g.embed * 2;
        bo = (size_t)g.embed * (g.q_dim() / tg::LG_QK) * tg::LG_Q4K_BYTES;
    } else {
        bq = 4 * (size_t)g.q_dim() * g.embed;
        bk = bv = 4 * (size_t)g.kv_dim() * g.embed;
        bo = 4 * (size_t)g.embed * g.q_dim();
    }
}

static int lg_attention(bool q4, const void *wq, const void *wk, const void *wv, const void *wo, const float *qnw,
                        const float *knw, float *kv_k, float *kv_v, const float *rope_cos, const float *rope_sin,
                        const float *input, float *output, const LgAttn &g) {
    if (!g.ok()) return set_err(TG_E_INVALID, "attention geometry");
    size_t bq, bk, bv, bo;
    lg_attn_wbytes(q4, g, bq, bk, bv, bo);
    const size_t nb = 4 * (size_t)g.hd;
    for (int pass = 0; pass < 2; pass++) {
        LgCarve c{pass ? g_lg_buf : nullptr};
        uint8_t *dq = c.take<uint8_t>(bq), *dk = c.take<uint8_t>(bk), *dv = c.take<uint8_t>(bv);
        uint8_t *dwo = c.take<uint8_t>(bo);
        float *dqn = c.take<float>(nb), *dkn = c.take<float>(nb);
        const LgAttnBufs b = lg_attn_bufs(c, g);
        if (!pass) {
            int rc = lg_reserve(c.off);
            if (rc) return rc;
            continue;
        }
        int rc;
        const uint8_t *pq, *pk, *pv, *po;
        const float *pqn, *pkn;
        if ((rc = lg_in(wq, bq, dq, &pq)) || (rc = lg_in(wk, bk, dk, &pk)) || (rc = lg_in(wv, bv, dv, &pv)) ||
            (rc = lg_in(wo, bo, dwo, &po)) || (rc = lg_in(qnw, nb, dqn, &pqn)) || (rc = lg_in(knw, nb, dkn, &pkn)) ||
            (rc = lg_h2d(b.x, input, 4 * (size_t)g.embed)) || (rc = lg_attn_in(g, b, kv_k, kv_v, rope_cos, rope_sin)) ||
            (rc = lg_attn_core(q4, pq, pk, pv, po, pqn, pkn, g, b)) || (rc = lg_attn_out(g, b, kv_k, kv_v)))
            return rc;
        return lg_finish(output, b.out, 4 * (size_t)g.embed);
    }
    return TG_OK;
}

extern "C" void tg_attention_decode(const float *wq, const float *wk, const float *wv, const float *wo,
                                    const float *q_norm_w, const float *k_norm_w, float *kv_k, float *kv_v,
                                    int kv_len, int kv_max, const float *rope_cos, const float *rope_sin,
                                    const float *input, float *output, int embed_dim, int n_heads, int n_kv_heads,
                                    int head_dim, int pos) {
    if (embed_dim <= 0) return;
    std::lock_guard<std::mutex> lk(g_lg_mu);
    const LgAttn g{embed_dim, n_heads, n_kv_heads, head_dim, kv_len, kv_max, pos};
    if (lg_attention(false, wq, wk, wv, wo, q_norm_w, k_norm_w, kv_k, kv_v, rope_cos, rope_sin, input, output, g)) {
        legacy_fail("tg_attention_decode", warned_attention_decode);
        fill_nan(output, embed_dim);
    }
}

extern "C" void tg_attention_decode_q4(const uint8_t *wq_q4, const uint8_t *wk_q4, const uint16_t *wv_f16,
                                       const uint8_t *wo_q4, const float *q_norm_w, const float *k_norm_w,
                                       float *kv_k, float *kv_v, int kv_len, int kv_max, const float *rope_cos,
                                       const float *rope_sin, const float *input, float *output, int embed_dim,
                                       int n_heads, int n_kv_heads, int head_dim, int pos) {
    if (embed_dim <= 0) return;
    std::lock_guard<std::mutex> lk(g_lg_mu);
    const LgAttn g{embed_dim, n_heads, n_kv_heads, head_dim, kv_len, kv_max, pos};
    if (lg_attention(true, wq_q4, wk_q4, wv_f16, wo_q4, q_norm_w, k_norm_w, kv_k, kv_v, rope_cos, rope_sin, input,
                     output, g)) {
        legacy_fail("tg_attention_decode_q4", warned_attention_decode_q4);
        fill_nan(output, embed_dim);
    }
}

// tg_transformer_layer (libtinygiant.c:662-702): RMS norm, f32 attention,
// x += attn; RMS norm, the experts' forward (down_is_f16[e] as the down
// format) accumulated from zero, x += moe.
static int lg_transformer_layer(const float *wq, const float *wk, const float *wv, const float *wo,
                                const float *attn_norm_w, const float *q_norm_w, const float *k_norm_w,
                                const float *ffn_norm_w, float *kv_k, float *kv_v, const float *rope_cos,
                                const float *rope_sin, const uint8_t **gate_ptrs, const uint8_t **up_ptrs,
                                const void **down_ptrs, const int *down_is_f16, const float *expert_weights,
                                int n_active, float *x, int inter, const LgAttn &g) {
    if (!g.ok() || inter <= 0 || n_active < 0) return set_err(TG_E_INVALID, "transformer layer geometry");
    size_t bq, bk, bv, bo;
    lg_attn_wbytes(false, g, bq, bk, bv, bo);
    const int embed = g.embed;
    const size_t gb = (size_t)inter * (embed / tg::LG_QK) * tg::LG_Q4K_BYTES;
    size_t dbmax = 0;
    bool all_q4k = tg::moe_q4k_ok(n_active, embed, inter);
    for (int e = 0; e < n_active; e++) {
        dbmax = std::max(dbmax, down_bytes(down_is_f16[e], embed, inter));
        all_q4k = all_q4k && down_is_f16[e] == 0;
    }
    // every expert Q4_K: the experts in three launches (as tg_moe_forward)
    const bool moe_all = all_q4k && lg_moe_all_enabled();
    const size_t nb = 4 * (size_t)g.hd, ev = 4 * (size_t)embed;
    for (int pass = 0; pass < 2; pass++) {
        LgCarve c{pass ? g_lg_buf : nullptr};
        uint8_t *dq = c.take<uint8_t>(bq), *dk = c.take<uint8_t>(bk), *dv = c.take<uint8_t>(bv);
        uint8_t *dwo = c.take<uint8_t>(bo);
        float *dqn = c.take<float>(nb), *dkn = c.take<float>(nb), *dan = c.take<float>(ev), *dfn = c.take<float>(ev);
        float *dx = c.take<float>(ev), *dmo = c.take<float>(ev);
        // one expert's staging (the per-expert loop)
        uint8_t *dg = c.take<uint8_t>(moe_all ? 0 : gb), *du = c.take<uint8_t>(moe_all ? 0 : gb);
        uint8_t *dd = c.take<uint8_t>(moe_all ? 0 : dbmax);
        const LgAttnBufs b = lg_attn_bufs(c, g);
        const LgExpertBufs eb = lg_expert_bufs(c, embed, inter);
        LgMoeAllBufs mb{};
        if (moe_all) mb = lg_moe_all_carve(c, n_active, embed, inter, 2 * gb + down_bytes(0, embed, inter));
        if (!pass) {
            int rc = lg_reserve(c.off);
            if (rc) return rc;
            continue;
        }
        hipStream_t st = g_lg_st;
        int rc;
        const uint8_t *pq, *pk, *pv, *po;
        const float *pqn, *pkn, *pan, *pfn;
        if ((rc = lg_in(wq, bq, dq, &pq)) || (rc = lg_in(wk, bk, dk, &pk)) || (rc = lg_in(wv, bv, dv, &pv)) ||
            (rc = lg_in(wo, bo, dwo, &po)) || (rc = lg_in(q_norm_w, nb, dqn, &pqn)) ||
            (rc = lg_in(k_norm_w, nb, dkn, &pkn)) || (rc = lg_in(attn_norm_w, ev, dan, &pan)) ||
            (rc = lg_in(ffn_norm_w, ev, dfn, &pfn)) || (rc = lg_h2d(dx, x, ev)) ||
            (rc = lg_attn_in(g, b, kv_k, kv_v, rope_cos, rope_sin)))
            return rc;
        PROFILED("lg_rms", st, tg::launch_rms_norm(dx, pan, b.x, embed, 1e-6f, st));
        if ((rc = lg_attn_core(false, pq, pk, pv, po, pqn, pkn, g, b))) return rc;
        PROFILED("lg_add", st, tg::launch_add_vec(dx, b.out, embed, st));
        PROFILED("lg_rms", st, tg::launch_rms_norm(dx, pfn, b.x, embed, 1e-6f, st));
        if (moe_all) {
            tg::LgMoeOps P;
            if ((rc = lg_moe_ops(n_active, gate_ptrs, up_ptrs, down_ptrs, expert_weights, gb, down_bytes(0, embed, inter),
                                 mb.stage, P)) ||
                (rc = lg_moe_run(P, n_active, b.x, dmo, embed, inter, eb, mb)))
                return rc;
        } else {
            HIP_TRY(hipMemsetAsync(dmo, 0, ev, st));  // moe_out starts at zero
            for (int e = 0; e < n_active; e++) {
                // one expert's operands at a time (a copy waits for the previous expert's kernels)
                const int fmt = down_is_f16[e];
                const uint8_t *pg, *pu, *pd;
                if ((rc = lg_in(gate_ptrs[e], gb, dg, &pg)) || (rc = lg_in(up_ptrs[e], gb, du, &pu)) ||
                    (rc = lg_in(down_ptrs[e], down_bytes(fmt, embed, inter), dd, &pd)) ||
                    (rc = lg_expert(pg, pu, pd, fmt, b.x, dmo, expert_weights[e], embed, inter, eb)))
                    return rc;
            }
        }
        PROFILED("lg_add", st, tg::launch_add_vec(dx, dmo, embed, st));
        if ((rc = lg_attn_out(g, b, kv_k, kv_v))) return rc;
        return lg_finish(x, dx, ev);
    }
    return TG_OK;
}

extern "C" void tg_transformer_layer(const float *wq, const float *wk, const float *wv, const float *wo,
                                     const float *attn_norm_w, const float *q_norm_w, const float *k_norm_w,
                                     const float *ffn_norm_w, float *kv_k, float *kv_v, int kv_len, int kv_max,
                                     const float *rope_cos, const float *rope_sin, const uint8_t **gate_ptrs,
                                     const uint8_t **up_ptrs, const void **down_ptrs, const int *down_is_f16,
                                     const float *expert_weights, int n_active, float *x, int embed_dim,
                                     int inter_dim, int n_heads, int n_kv_heads, int head_dim, int pos) {
    if (embed_dim <= 0) return;
    std::lock_guard<std::mutex> lk(g_lg_mu);
    const LgAttn g{embed_dim, n_heads, n_kv_heads, head_dim, kv_len, kv_max, pos};
    if (lg_transformer_layer(wq, wk, wv, wo, attn_norm_w, q_norm_w, k_norm_w, ffn_norm_w, kv_k, kv_v, rope_cos,
                             rope_sin, gate_ptrs, up_ptrs, down_ptrs, down_is_f16, expert_weights, n_active, x,
                             inter_dim, g)) {
        legacy_fail("tg_transformer_layer", warned_transformer_layer);
        fill_nan(x, embed_dim);
    }
}


// ------------------------------------------------------------- output head
// The step after the layers (engine.py:262-266,359): logits = W ·
// rms_norm(x, output_norm) with W [vocab][embed] fp32, then the greedy token
// argmax(logits).  The reference keeps W in a numpy array and multiplies with
// `@`; here W stays resident in HBM behind a handle, the product follows the
// reference's own fp32 matvec order (tg_f32_matvec, libtinygiant.c:299-318)
// and the norm tg_rms_norm's (:322-340).
struct tg_sampler;
static void sampler_free(tg_sampler *s);

struct tg_head {
    int vocab, embed, dev;
    float *W, *nw, *x, *xn, *logits, *pv;
    int *pi, *tok;
    tg_sampler *smp;  // created by the first tg_head_sample
};

static void head_free(tg_head *h) {
    if (!h) return;
    sampler_free(h->smp);
    for (void *p : {(void *)h->W, (void *)h->nw, (void *)h->x, (void *)h->xn, (void *)h->logits, (void *)h->pv,
                    (void *)h->pi, (void *)h->tok})
        if (p) (void)hipFree(p);
    delete h;
}

extern "C" tg_head *tg_head_create(const float *W, const float *norm_w, int vocab, int embed) {
    if (!W || !norm_w || vocab <= 0 || embed <= 0) {
        set_err(TG_E_INVALID, "tg_head_create: vocab %d, embed %d", vocab, embed);
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_lg_mu);
    if (lg_reserve(0)) return nullptr;
    tg_head *h = new tg_head{vocab, embed, g_lg_dev, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                             nullptr, nullptr};
    const size_t wb = sizeof(float) * (size_t)vocab * embed, eb = sizeof(float) * (size_t)embed;
    auto alloc = [&](void **p, size_t n) { return hipMalloc(p, n) == hipSuccess; };
    if (!alloc((void **)&h->W, wb) || !alloc((void **)&h->nw, eb) || !alloc((void **)&h->x, eb) ||
        !alloc((void **)&h->xn, eb) || !alloc((void **)&h->logits, sizeof(float) * (size_t)vocab) ||
        !alloc((void **)&h->pv, sizeof(float) * tg::ARGMAX_BLOCKS) ||
        !alloc((void **)&h->pi, sizeof(int) * tg::ARGMAX_BLOCKS) || !alloc((void **)&h->tok, sizeof(int))) {
        (void)hipGetLastError();
        head_free(h);
        set_err(TG_E_NOMEM, "tg_head_create: %zu bytes of output weights", wb);
        return nullptr;
    }
    if (hipMemcpy(h->W, W, wb, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(h->nw, norm_w, eb, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipGetLastError();
        head_free(h);
        set_err(TG_E_HIP, "tg_head_create: copy of the output weights failed");
        return nullptr;
    }
    return h;
}

extern "C" void tg_head_destroy(tg_head *h) { head_free(h); }

// x (embed floats, host) -> logits (vocab floats, host; may be null) and the
// greedy token.  Returns 0 or a negative TG_E_* code.
extern "C" int tg_head_forward(tg_head *h, const float *x, float eps, float *logits, int32_t *token) {
    if (!h || !x || !token) return set_err(TG_E_INVALID, "tg_head_forward: null handle, input or token");
    std::lock_guard<std::mutex> lk(g_lg_mu);
    int rc = lg_reserve(0);
    if (rc) return rc;
    if (g_lg_dev != h->dev) return set_err(TG_E_INVALID, "tg_head_forward: handle of device %d", h->dev);
    hipStream_t st = g_lg_st;
    const size_t eb = sizeof(float) * (size_t)h->embed;
    if ((rc = lg_h2d(h->x, x, eb))) return rc;
    PROFILED("head_rms", st, tg::launch_rms_norm(h->x, h->nw, h->xn, h->embed, eps, st));
    PROFILED("head_mv", st, tg::launch_matvec_two_acc(h->W, false, h->xn, h->logits, h->vocab, h->embed, st));
    PROFILED("head_argmax", st, tg::launch_argmax(h->logits, h->vocab, h->pv, h->pi, h->tok, st));
    if (logits) HIP_TRY(hipMemcpyAsync(logits, h->logits, sizeof(float) * (size_t)h->vocab, hipMemcpyDeviceToHost, st));
    return lg_finish(token, h->tok, sizeof(int32_t));
}

// ------------------------------------------------------------- sampling
// engine.py:348-359: the next token from the logits, by temperature and
// top-p (tg_sample.hip) when temperature > 0, else the greedy argmax.  The
// reference draws with np.random.choice; the caller passes that draw's
// uniform u in [0, 1) (choice takes one RandomState.random_sample() per
// draw), so the same u gives the reference's token.  Device buffers for one
// vocabulary are allocated once per sampler.
struct tg_sampler {
    int vocab, dev;
    tg::SmpBufs b;
    float *dl;            // logits copied from the host
    float *pv;            // greedy argmax partials
    int *pi, *tok;
    void *mem;
    tg::SmpCtl *hctl;     // pinned host copy of b.ctl
};

static void sampler_free(tg_sampler *s) {
    if (!s) return;
    if (s->mem) (void)hipFree(s->mem);
    if (s->hctl) (void)hipHostFree(s->hctl);
    delete s;
}

// Caller holds g_lg_mu and has run lg_reserve.
static int sampler_new(int vocab, tg_sampler **out) {
    *out = nullptr;
    if (vocab <= 0 || vocab > tg::SMP_VMAX)
        return set_err(TG_E_INVALID, "sampler: vocab %d outside 1..%d", vocab, tg::SMP_VMAX);
    static bool prepared = false;
    if (!prepared) {
        if (tg::sample_prepare() != hipSuccess) {
            (void)hipGetLastError();
            return set_err(TG_E_HIP, "sampler: LDS attribute of the sort kernel");
        }
        prepared = true;
    }
    tg_sampler *s = new tg_sampler{};
    s->vocab = vocab;
    s->dev = g_lg_dev;
    size_t nk = 16384;
    while (nk < (size_t)vocab) nk <<= 1;
    const size_t V = (size_t)vocab;
    LgCarve c{nullptr};
    for (int pass = 0; pass < 2; pass++) {
        c = LgCarve{pass ? (uint8_t *)s->mem : nullptr};
        s->b.pmax = c.take<float>(sizeof(float) * 256);
        s->b.pbad = c.take<int>(sizeof(int) * 256);
        s->b.p = c.take<float>(sizeof(float) * V);
        s->b.q = c.take<float>(sizeof(float) * V);
        s->b.sums = c.take<float>(sizeof(float) * 64);
        s->b.hcnt = c.take<uint32_t>(sizeof(uint32_t) * tg::SMP_BUCKETS);
        s->b.hmass = c.take<unsigned long long>(sizeof(unsigned long long) * tg::SMP_BUCKETS);
        s->b.keys = c.take<unsigned long long>(sizeof(unsigned long long) * nk);
        s->b.sq = c.take<float>(sizeof(float) * V);
        s->b.sid = c.take<uint32_t>(sizeof(uint32_t) * V);
        s->b.ctl = c.take<tg::SmpCtl>(sizeof(tg::SmpCtl));
        s->dl = c.take<float>(sizeof(float) * V);
        s->pv = c.take<float>(sizeof(float) * tg::ARGMAX_BLOCKS);
        s->pi = c.take<int>(sizeof(int) * tg::ARGMAX_BLOCKS);
        s->tok = c.take<int>(sizeof(int));
        if (!pass && (hipMalloc(&s->mem, c.off) != hipSuccess ||
                      hipHostMalloc((void **)&s->hctl, sizeof(tg::SmpCtl), hipHostMallocDefault) != hipSuccess)) {
            (void)hipGetLastError();
            sampler_free(s);
            return set_err(TG_E_NOMEM, "sampler: %zu bytes for vocab %d", c.off, vocab);
        }
    }
    *out = s;
    return TG_OK;
}

// Caller holds g_lg_mu; dl = device logits of s->vocab values.
static int sampler_run(tg_sampler *s, const float *dl, float temperature, double top_p, double u, int32_t *token,
                       float *probs) {
    hipStream_t st = g_lg_st;
    if (!(temperature > 0.0f)) {  // engine.py:358-359 (a NaN temperature is not > 0 either)
        PROFILED("sample_argmax", st, tg::launch_argmax(dl, s->vocab, s->pv, s->pi, s->tok, st));
        return lg_finish(token, s->tok, sizeof(int32_t));
    }
    if (!(u >= 0.0 && u < 1.0)) return set_err(TG_E_INVALID, "sample: u = %g is not in [0, 1)", u);
    PROFILED("sample", st, tg::launch_sample_main(s->b, dl, s->vocab, temperature, top_p, u, st));
    HIP_TRY(hipMemcpyAsync(s->hctl, s->b.ctl, sizeof(tg::SmpCtl), hipMemcpyDeviceToHost, st));
    if (probs) HIP_TRY(hipMemcpyAsync(probs, s->b.q, sizeof(float) * (size_t)s->vocab, hipMemcpyDeviceToHost, st));
    int rc = lg_sync();
    if (rc) return rc;
    tg::SmpCtl c = *s->hctl;
    if (c.bad || c.status == tg::SMP_ST_INPUT)
        return set_err(TG_E_INVALID, "sample: the logits hold NaN or +inf, or every logit is -inf");
    if (c.large) {
        PROFILED("sample_large", st, tg::launch_sample_large(s->b, s->vocab, (int)c.C, top_p, u, st));
        HIP_TRY(hipMemcpyAsync(s->hctl, s->b.ctl, sizeof(tg::SmpCtl), hipMemcpyDeviceToHost, st));
        if ((rc = lg_sync())) return rc;
        c = *s->hctl;
    }
    if (c.status != tg::SMP_ST_OK || c.token < 0 || c.token >= s->vocab)
        return set_err(TG_E_HIP, "sample: device status %d, token %d, %u candidates", c.status, c.token, c.C);
    *token = c.token;
    return TG_OK;
}

extern "C" tg_sampler *tg_sampler_create(int vocab) {
    std::lock_guard<std::mutex> lk(g_lg_mu);
    if (vocab <= 0 || vocab > tg::SMP_VMAX) {
        set_err(TG_E_INVALID, "tg_sampler_create: vocab %d outside 1..%d", vocab, tg::SMP_VMAX);
        return nullptr;
    }
    tg_sampler *s = nullptr;
    if (lg_reserve(0) || sampler_new(vocab, &s)) return nullptr;
    return s;
}

extern "C" void tg_sampler_destroy(tg_sampler *s) { sampler_free(s); }

extern "C" int tg_sampler_run(tg_sampler *s, const float *logits, int logits_on_device, float temperature,
                              double top_p, double u, int32_t *token, float *probs) {
    if (!s || !logits || !token) return set_err(TG_E_INVALID, "tg_sampler_run: null handle, logits or token");
    std::lock_guard<std::mutex> lk(g_lg_mu);
    int rc = lg_reserve(0);
    if (rc) return rc;
    if (g_lg_dev != s->dev) return set_err(TG_E_INVALID, "tg_sampler_run: handle of device %d", s->dev);
    const float *dl = logits;
    if (!logits_on_device) {
        if ((rc = lg_h2d(s->dl, logits, sizeof(float) * (size_t)s->vocab))) return rc;
        dl = s->dl;
    }
    return sampler_run(s, dl, temperature, top_p, u, token, probs);
}

// The head's logits sampled on the device: x (embed floats, host) -> token.
extern "C" int tg_head_sample(tg_head *h, const float *x, float eps, float temperature, double top_p, double u,
                              float *logits, int32_t *token) {
    if (!h || !x || !token) return set_err(TG_E_INVALID, "tg_head_sample: null handle, input or token");
    std::lock_guard<std::mutex> lk(g_lg_mu);
    int rc = lg_reserve(0);
    if (rc) return rc;
    if (g_lg_dev != h->dev) return set_err(TG_E_INVALID, "tg_head_sample: handle of device %d", h->dev);
    if (temperature > 0.0f && !(u >= 0.0 && u < 1.0))
        return set_err(TG_E_INVALID, "tg_head_sample: u = %g is not in [0, 1)", u);
    if (!h->smp && (rc = sampler_new(h->vocab, &h->smp))) return rc;
    hipStream_t st = g_lg_st;
    const size_t eb = sizeof(float) * (size_t)h->embed;
    if ((rc = lg_h2d(h->x, x, eb))) return rc;
    PROFILED("head_rms", st, tg::launch_rms_norm(h->x, h->nw, h->xn, h->embed, eps, st));
    PROFILED("head_mv", st, tg::launch_matvec_two_acc(h->W, false, h->xn, h->logits, h->vocab, h->embed, st));
    if (logits) HIP_TRY(hipMemcpyAsync(logits, h->logits, sizeof(float) * (size_t)h->vocab, hipMemcpyDeviceToHost, st));
    return sampler_run(h->smp, h->logits, temperature, top_p, u, token, nullptr);
}
