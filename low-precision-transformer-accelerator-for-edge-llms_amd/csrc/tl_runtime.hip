// tl_runtime.hip -- C++ runtime behind the C-ABI of include/tl_int8.h.
//
// Owns the device copy of the quantized model, the INT8 KV cache, the
// workspaces and one HIP stream per handle, and sequences the kernels of
// tl_kernels.hip into the reference's decoder-layer / generation schedule
// (model/tinyllama_gemm_int8.py:256-281, 437-467, 629-685;
// rtl/control/layer_controller.sv block order).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <mutex>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "tl_int8.h"
#include "tl_internal.h"

using namespace tl;

namespace {

struct LayerDev {
    int8_t* wqkv = nullptr;  // [D + 2 KVD][D]  q rows, then k rows, then v rows
    float* sqkv = nullptr;
    int8_t* wo = nullptr;
    float* so = nullptr;
    int8_t* wg = nullptr;
    float* sg = nullptr;
    int8_t* wu = nullptr;
    float* su = nullptr;
    int8_t* wd = nullptr;
    float* sd = nullptr;
    float* g_in = nullptr;
    float* g_post = nullptr;
    // packed copies (MFMA operand blocks) read by the M <= 32 GEMMs of
    // batched decode; null when the geometry has no 32-multiple shapes
    int8_t* wqkv_p = nullptr;
    int8_t* wo_p = nullptr;
    int8_t* wg_p = nullptr;
    int8_t* wu_p = nullptr;
    int8_t* wd_p = nullptr;
};

constexpr int kWatchDepth = 3;      // decode steps (or prefill layers) in flight while the host watches
                                    // for EOS and a host abort

struct ProfEvent {
    int kclass;
    hipEvent_t start, stop;
    double bytes;
};

thread_local std::string g_create_error;

// ---- fixed scratch of tl_gemm_i8_noalloc ---------------------------------------
// One copy per GPU of this file-scope device array: the split-K partial tiles
// of the small-M GEMM (tiles x slices x 1024 int32 with tiles x slices < 512,
// so at most 2 MiB) and 256 per-tile arrival counters.  Host code never
// passes the array's name: tl_create looks up the current device's copy with
// hipGetSymbolAddress once per device and every handle keeps that address.
constexpr size_t kNoAllocPartials = (size_t)512 * 1024;   // int32 elements
constexpr int32_t kNoAllocCounters = 256;
static __device__ __align__(256) int32_t scratch[kNoAllocPartials + kNoAllocCounters];

// Every call on a GPU shares that GPU's copy, so calls from different handles
// (different streams, different host threads) are put in order: under
// g_scratch_mu a call makes its stream wait for the device's event, launches,
// and records the event again, so its kernels start after the previous
// call's have finished.  The event is created with the address lookup (at
// tl_create), so the entry point itself creates nothing.
std::mutex g_scratch_mu;
std::vector<void*> g_scratch_dev;        // device address of `scratch`, by device ordinal
std::vector<hipEvent_t> g_scratch_done;  // last use of that device's copy

hipError_t scratch_address(int dev, void** out, hipEvent_t* done) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if ((int)g_scratch_dev.size() <= dev) {
        g_scratch_dev.resize(dev + 1, nullptr);
        g_scratch_done.resize(dev + 1, nullptr);
    }
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        hipEvent_t ev = nullptr;
        if ((e = hipEventCreateWithFlags(&ev, hipEventDisableTiming)) != hipSuccess) return e;
        g_scratch_dev[dev] = p;
        g_scratch_done[dev] = ev;
    }
    *out = g_scratch_dev[dev];
    *done = g_scratch_done[dev];
    return hipSuccess;
}

}  // namespace

struct tl_handle {
    tl_config cfg{};
    int32_t max_seqs = 0;
    int32_t max_rows = 0;
    int device = 0;
    hipStream_t stream = nullptr;
    PwPlan plan{};
    int32_t D = 0, F = 0, KVD = 0, QKV = 0;

    std::vector<LayerDev> layers;
    int8_t* lm_w = nullptr;
    int8_t* lm_wp = nullptr;      // packed copy of lm_w (batched decode LM head), or null
    float* lm_s = nullptr;
    float* g_final = nullptr;
    int8_t* emb = nullptr;
    float* emb_s = nullptr;
    float* rope_cos = nullptr;
    float* rope_sin = nullptr;
    int32_t rope_n = 0;
    float* att_max = nullptr;   // [max rows][n_heads]: each head's max |attention output| (batched decode)
    int32_t* pf_sink = nullptr; // written by the L2 prefetch workgroups only if their loads XOR to a magic value
    float* kv_sk = nullptr;
    float* kv_sv = nullptr;
    KvGeom kv{};

    // workspaces, [max_rows] rows each
    float* x = nullptr;
    float* qkv = nullptr;
    int8_t* a8 = nullptr;
    double* as = nullptr;
    int8_t* q8 = nullptr;
    double* qs = nullptr;
    float* att = nullptr;
    float* hid = nullptr;
    float* logits = nullptr;      // [max_seqs][V]
    int32_t* row_seq = nullptr;
    int32_t* row_pos = nullptr;
    int32_t* tokens = nullptr;    // [max_rows]
    int8_t* kv_stage = nullptr;   // [2][max_pos][64] staging of tl_kv_write / tl_kv_read rows
    int32_t* noalloc_scratch = nullptr;   // this device's copy of `scratch` (tl_gemm_i8_noalloc)
    hipEvent_t noalloc_done = nullptr;    // the device's event ordering the calls that use it
    float* fscratch = nullptr;    // small scratch
    unsigned long long* op_key = nullptr;  // argmax slot of the standalone LM-head operator
    unsigned long long* lm_wg_keys = nullptr;  // [vocab / 4] batch-1 LM head: argmax key per workgroup
    int32_t* partials = nullptr;
    int32_t* racc = nullptr;      // [32][D] integer sums of the K-sliced batched-decode down GEMM; zero
                                  // between uses (the fold prologue clears what it read)
    size_t racc_cap = 0;          // int32 elements
    int32_t* qacc = nullptr;      // [32][QKV] integer sums of the K-sliced batched-decode Q|K|V GEMM, read
                                  // by the attention kernel; zero between uses (the attention output's
                                  // quantization clears them)
    size_t qacc_cap = 0;          // int32 elements
    unsigned* qmax = nullptr;     // [max_rows][kQmaxStride] prefill: max|q| of each rotated Q row (float bits, element 0)
                                  // from the fused Q|K|V GEMM; zero between uses (the attention output's
                                  // quantization clears them)
    unsigned* tile_ctr = nullptr;         // [kSkinnyTiles] arrival counters of the small-M GEMM, zero between launches
    size_t partial_cap = 0;       // int32 elements

    // per-sequence generation state
    unsigned long long* keys = nullptr;
    int32_t* token_cur = nullptr;
    int32_t* cursor = nullptr;
    int32_t* n_gen = nullptr;
    int32_t* eos_id = nullptr;       // [max_seqs] EOS id the captured step checks (< 0: none)
    int32_t* stopped = nullptr;      // [max_seqs] set on the device when the EOS token is recorded
    int32_t* tokens_out = nullptr;   // [max_seqs][max_pos]
    float* logit_out = nullptr;      // [max_seqs][max_pos]
    std::vector<int32_t> host_cursor;
    int32_t stop_state[2] = {-1, 0};  // host words copied into eos_id / stopped
    // pinned host words the device reads and writes: [0] the abort word the
    // token bookkeeping kernel checks every step, [1 + seq] the mirror of
    // stopped[seq] it writes (1 EOS, 2 host abort)
    int32_t* ctl_host = nullptr;      // host view
    int32_t* ctl_dev = nullptr;       // device view of the same words
    hipEvent_t watch_ev[kWatchDepth] = {};
    std::vector<int32_t> host_ngen;

    std::vector<void*> allocs;
    std::string err;


    bool batch_kslice = true;             // batched decode: K-sliced down GEMM folded by the next RMSNorm
                                          // row prologue (TL_BATCH_KSLICE=0 turns it off)
    const float* racc_res_ws = nullptr;   // racc holds a down projection's sums (these weight scales) that
                                          // the next RMSNorm prologue adds to h->x
    bool racc_clean = true;               // false from an EPI_ACC launch until its fold has run
    bool qkv_kslice = true;               // batched decode: K-sliced Q|K|V GEMM whose sums the attention
                                          // kernel dequantizes (TL_BATCH_QKV_KSLICE=0 turns it off)
    bool qacc_clean = true;               // false from a Q|K|V EPI_ACC launch until qacc is cleared
    bool o_fuse = true;                   // batched decode: the O GEMM K-sliced, quantizing the attention output itself
                                          // at the row maxima the attention kernel leaves; its sums folded by the
                                          // post-attention RMSNorm (TL_BATCH_O_FUSE=0 turns it off)
    bool qmax_clean = true;               // false from a fused Q|K|V GEMM until qmax is cleared
    bool rows_one_seq = false;            // the uploaded rows are one sequence at rows_pos0 + r
    int32_t rows_seq = 0, rows_pos0 = 0;
    std::vector<hipGraphExec_t> graphs;   // captured batch-1 decode step per sequence
    std::vector<hipGraphExec_t> batch_graphs;   // captured batched decode step, by batch size

    bool profiling = false;
    // decode timeline: while ts_on, the launches of a step take consecutive
    // regions of ts_buf for their wavefronts' clock stamps
    struct TsSlot {
        int kclass;
        size_t off;       // u64 elements into ts_buf
        int64_t waves;
    };
    bool ts_on = false;
    bool ts_overflow = false;
    unsigned long long* ts_buf = nullptr;
    size_t ts_cap = 0;
    size_t ts_used = 0;
    std::vector<TsSlot> ts_slots;
    std::vector<ProfEvent> prof_pending;
    std::vector<hipEvent_t> event_pool;
    int64_t prof_count[TL_K_COUNT] = {};
    double prof_ms[TL_K_COUNT] = {};
    double prof_bytes[TL_K_COUNT] = {};
};

namespace {

int fail(tl_handle* h, int32_t code, const std::string& msg) {
    if (h) h->err = msg;
    else g_create_error = msg;
    return code;
}

#define TL_HIP(h, expr)                                                                     \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess)                                                               \
            return fail((h), TL_ERR_INTERNAL, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

#define TL_REQ(h, cond, msg)                                               \
    do {                                                                   \
        if (!(cond)) return fail((h), TL_ERR_BAD_DESCRIPTOR, (msg));       \
    } while (0)

template <typename T>
hipError_t dalloc(tl_handle* h, T** p, size_t count) {
    void* q = nullptr;
    hipError_t e = hipMalloc(&q, std::max<size_t>(count, 1) * sizeof(T));
    if (e == hipSuccess) {
        h->allocs.push_back(q);
        *p = (T*)q;
    }
    return e;
}

}  // namespace

KernelTiming& tl::kernel_timing() {
    thread_local KernelTiming t;
    return t;
}

namespace {

hipEvent_t take_event(tl_handle* h) {
    if (!h->event_pool.empty()) {
        hipEvent_t e = h->event_pool.back();
        h->event_pool.pop_back();
        return e;
    }
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// optional per-kernel-class timing: the kernels of one operation carry the
// start / stop events themselves (see TL_KLAUNCH)
struct Prof {
    tl_handle* h;
    int kc;
    double bytes;
    bool on;
    hipEvent_t a = nullptr, b = nullptr;
    KernelTiming saved;
    Prof(tl_handle* hh, int k, double bb, bool allow = true) : h(hh), kc(k), bytes(bb), on(hh->profiling && allow) {
        if (!on) return;
        a = take_event(h);
        b = take_event(h);
        if (!a || !b) return;
        saved = kernel_timing();
        kernel_timing() = KernelTiming{a, b, false};
    }
    ~Prof() {
        if (!on) return;
        if (a && b) {
            const bool used = kernel_timing().used;
            kernel_timing() = saved;
            if (used) {
                h->prof_pending.push_back({kc, a, b, bytes});
                return;
            }
        }
        if (a) h->event_pool.push_back(a);
        if (b) h->event_pool.push_back(b);
    }
};

void harvest_profile(tl_handle* h) {
    if (h->prof_pending.empty()) return;
    (void)hipStreamSynchronize(h->stream);   // a failed step shows as failed elapsed-time reads below
    for (auto& p : h->prof_pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
            h->prof_count[p.kclass] += 1;
            h->prof_ms[p.kclass] += ms;
            h->prof_bytes[p.kclass] += p.bytes;
        }
        h->event_pool.push_back(p.start);
        h->event_pool.push_back(p.stop);
    }
    h->prof_pending.clear();
}

hipError_t copy_in(tl_handle* h, void* dst, const void* src, size_t bytes, int32_t src_mem) {
    return hipMemcpyAsync(dst, src, bytes, src_mem == TL_MEM_DEVICE ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                          h->stream);
}

// default RoPE table following TL:59-66 step by step in float32
void default_rope(int32_t n_pos, float theta, std::vector<float>& c, std::vector<float>& s) {
    float inv[kHeadDim / 2];
    for (int i = 0; i < kHeadDim / 2; i++) {
        const float e = (float)(2 * i) / (float)kHeadDim;
        inv[i] = 1.0f / powf(theta, e);
    }
    c.resize((size_t)n_pos * kHeadDim);
    s.resize((size_t)n_pos * kHeadDim);
    for (int p = 0; p < n_pos; p++)
        for (int d = 0; d < kHeadDim; d++) {
            const float a = (float)p * inv[d % (kHeadDim / 2)];
            c[(size_t)p * kHeadDim + d] = (float)cos((double)a);
            s[(size_t)p * kHeadDim + d] = (float)sin((double)a);
        }
}

int32_t check_launch(tl_handle* h, hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(h, TL_ERR_INTERNAL, std::string(what) + ": " + hipGetErrorString(e));
    return TL_OK;
}

#define TL_LAUNCH(h, expr)                                   \
    do {                                                     \
        int32_t r_ = check_launch((h), (expr), #expr);       \
        if (r_) return r_;                                   \
    } while (0)

int32_t finish(tl_handle* h) {
    hipError_t e = hipStreamSynchronize(h->stream);
    if (e != hipSuccess) return fail(h, TL_ERR_INTERNAL, std::string("stream: ") + hipGetErrorString(e));
    if (h->profiling) harvest_profile(h);
    return TL_OK;
}

// ---- GEMM dispatch: M == 1 uses the GEMV kernels, M > 1 the MFMA kernels ----
int32_t ensure_partials(tl_handle* h, size_t need) {
    if (need <= h->partial_cap) return TL_OK;
    if (h->partials) {
        (void)hipFree(h->partials);
        h->allocs.erase(std::remove(h->allocs.begin(), h->allocs.end(), (void*)h->partials), h->allocs.end());
        h->partials = nullptr;
    }
    TL_HIP(h, dalloc(h, &h->partials, need));
    h->partial_cap = need;
    return TL_OK;
}

// caller-fixed scratch for the split-K small-M GEMM (the no-allocation entry
// point): partial tiles and per-tile arrival counters
struct FixedScratch {
    int32_t* part;
    size_t part_cap;      // int32 elements
    unsigned* ctr;
    int32_t ctr_cap;      // counters
};

// wavefronts per workgroup of the packed M <= 32 GEMM: with 8 (8 chunks of
// 32 bytes each) the gate/up GEMM took 225 against 273 us per batched step at
// 32 x 2048, while Q|K|V, O and down were 4-12 % slower than with 16
static int rows32_waves(int epi) {
    return epi == EPI_GLU ? 8 : 16;
}

int32_t run_gemm(tl_handle* h, int epi, GemmArgs a, int kclass, const FixedScratch* fx = nullptr) {
    const int nb = epi == EPI_GLU ? 2 : 1;
    const bool prof_ok = fx == nullptr;   // profiling events are allocations
    const double bytes = (double)a.m * a.k + (double)nb * a.n * a.k + (double)a.m * a.n * 4.0;
    if (a.ap) {
        // A was written in the packed operand layout for this GEMM
        Prof p(h, kclass, bytes, prof_ok);
        TL_LAUNCH(h, launch_gemm_pk(h->stream, epi, a));
        return TL_OK;
    }
    if (a.m >= 64) {
        // 32x32x32 MFMA tiles: the 64 x 64 block-tiled kernel with 128-byte K
        // stages when K is a multiple of 128, else the two-K-slice kernel
        const bool tile = a.k % 128 == 0;
        a.k_split = a.k;
        Prof p(h, kclass, bytes, prof_ok);
        TL_LAUNCH(h, launch_gemm32(h->stream, epi, a, tile));
        return TL_OK;
    }
    if (a.m <= 32 && a.wp && (epi != EPI_GLU || (a.wp2 && a.k <= 2048)) && a.k % 64 == 0 && a.k <= 6144 &&
        a.n % 32 == 0) {
        // batched decode on the packed weight copies: one 16-wavefront
        // workgroup per 32 output columns, every weight load a coalesced 1 KiB
        // (measured faster than splitting K over workgroups: the cross-XCD
        // reduction of the partial tiles costs more than the added bandwidth)
        Prof p(h, kclass, bytes, prof_ok);
        TL_LAUNCH(h, launch_gemm_rows32(h->stream, epi, a, rows32_waves(epi)));
        return TL_OK;
    }
    a.wp = a.wp2 = nullptr;
    if (a.m <= 32 && a.k % 64 == 0 && a.k <= 6144) {
        // batched decode: one 32-row MFMA tile per 32 output columns, K split
        // over enough workgroups to cover the chip, reduced in the kernel
        const int tiles = (a.n + 31) / 32, kch = a.k / 32;
        int slices = 1;
        while (tiles * slices < 256 && kch / (4 * slices * 2) >= 2 && slices < kSkinnyMaxSlices) slices *= 2;
        if (tiles > kSkinnyTiles) slices = 1;
        int32_t* part = h->partials;
        unsigned* ctr = h->tile_ctr;
        const bool skinny = a.k > 2048;
        if (fx) {
            if (skinny && slices > 1) {
                if ((size_t)tiles * slices * nb * 1024 > fx->part_cap || tiles > fx->ctr_cap)
                    return fail(h, TL_ERR_UNSUPPORTED, "GEMM needs more split-K scratch than the fixed " +
                                                           std::to_string(fx->part_cap * 4) + "-byte buffer holds");
                // the counters start at zero (the last workgroup of a tile resets its own)
                TL_LAUNCH(h, launch_fill_u32(h->stream, fx->ctr, tiles, 0u));
            }
            part = fx->part;
            ctr = fx->ctr;
        } else if (slices > 1) {
            int32_t r = ensure_partials(h, (size_t)tiles * slices * nb * 1024);
            if (r) return r;
            part = h->partials;
        }
        Prof p(h, kclass, bytes, prof_ok);
        if (skinny)
            TL_LAUNCH(h, launch_gemm_skinny(h->stream, epi, a, slices, part, ctr));
        else TL_LAUNCH(h, launch_gemm_rows32(h->stream, epi, a));
        return TL_OK;
    }
    // small M (33..63 rows): 16x16x64 tiles, split K until the output tiles
    // plus K splits cover the chip
    const int bm = a.m <= 32 ? 32 : 64;
    const int64_t tiles = (int64_t)((a.m + bm - 1) / bm) * ((a.n + 63) / 64);
    int splits = 1;
    while (tiles * splits < 512 && a.k / (64 * splits * 2) >= 4 && splits < 16) splits *= 2;
    if (epi == EPI_RAW) splits = 1;
    a.k_split = ((a.k / 64 + splits - 1) / splits) * 64;
    splits = (a.k + a.k_split - 1) / a.k_split;
    if (splits > 1) {
        if (fx) return fail(h, TL_ERR_UNSUPPORTED, "split GEMM of 33..63 rows has no fixed-scratch form");
        int32_t r = ensure_partials(h, (size_t)splits * nb * a.m * a.n);
        if (r) return r;
        a.acc = h->partials;
    }
    Prof p(h, kclass, bytes, prof_ok);
    TL_LAUNCH(h, launch_gemm(h->stream, epi, a, splits));
    if (splits > 1) TL_LAUNCH(h, launch_gemm_reduce(h->stream, epi, a, splits));
    return TL_OK;
}

int32_t linear(tl_handle* h, int epi, int rows, const int8_t* x8, const double* xs, const int8_t* w,
               const float* ws, const int8_t* w2, const float* ws2, int32_t n, int32_t k,
               const float* residual, float* y, int kclass, const int8_t* wp = nullptr,
               const int8_t* wp2 = nullptr, bool a_packed = false) {
    if (rows == 1) {
        GemvArgs g{};
        g.w = w; g.w2 = w2; g.ws = ws; g.ws2 = ws2; g.x = x8; g.xs = xs;
        g.residual = residual; g.y = y; g.n = n; g.k = k;
        const double bytes = (double)(w2 ? 2 : 1) * ((double)n * k + n * 4.0) + k + n * 4.0 + (residual ? n * 4.0 : 0.0);
        Prof p(h, kclass, bytes);
        TL_LAUNCH(h, launch_gemv(h->stream, epi, g));
        return TL_OK;
    }
    GemmArgs a{};
    a.a = x8; a.w = w; a.w2 = w2; a.as = xs; a.ws = ws; a.ws2 = ws2;
    a.residual = residual; a.y = y; a.m = rows; a.n = n; a.k = k; a.wp = wp; a.wp2 = wp2;
    a.ap = a_packed ? x8 : nullptr;
    // multi-row GEMMs keep their role's class (Q|K|V, O, gate/up, down, LM head)
    return run_gemm(h, epi, a, kclass);
}

RowMap rowmap(tl_handle* h) { return RowMap{h->row_seq, h->row_pos}; }

// causal attention of the uploaded rows: MFMA tiles when the rows are one
// sequence (prefill), else one workgroup per (row, KV head)
hipError_t rows_attention(tl_handle* h, const int8_t* q8, const double* q_scale, int32_t rows, int32_t layer,
                          float* out, int32_t max_t) {
    const tl_config& c = h->cfg;
    if (h->rows_one_seq && h->rows_pos0 + rows <= kTileMaxKeys)
        return launch_attention_tiles(h->stream, q8, q_scale, rows, c.n_heads, c.n_kv_heads, h->rows_seq, h->rows_pos0,
                                      h->kv, layer, h->kv_sk, h->kv_sv, out);
    return launch_attention(h->stream, q8, q_scale, rows, c.n_heads, c.n_kv_heads, rowmap(h), h->kv, layer, h->kv_sk,
                            h->kv_sv, out, max_t);
}

// stamp region for one launch of `waves` wavefronts (null unless capturing a
// timeline step)
unsigned long long* ts_take(tl_handle* h, int kclass, int64_t waves) {
    if (!h->ts_on || waves <= 0) return nullptr;
    if (h->ts_used + 2 * (size_t)waves > h->ts_cap) {
        h->ts_overflow = true;
        return nullptr;
    }
    unsigned long long* p = h->ts_buf + h->ts_used;
    h->ts_slots.push_back({kclass, h->ts_used, waves});
    h->ts_used += 2 * (size_t)waves;
    return p;
}

GemvArgs gemv_args(const tl_handle* h) {
    GemvArgs g{};
    g.eps = h->cfg.rms_eps;
    g.plan = h->plan;
    return g;
}

// one decoder layer (GI:256-281) for a single row (batch-1 decode or a
// one-token prefill) as five fused kernels; the row's sequence and position
// are in h->row_seq[0] / h->row_pos[0]; max_t bounds pos + 1
int32_t layer_row1(tl_handle* h, int32_t layer, int32_t max_t) {
    const tl_config& c = h->cfg;
    const LayerDev& L = h->layers[layer];
    const int D = h->D, F = h->F, QKV = h->QKV;
    {
        GemvArgs g = gemv_args(h);
        g.xf = h->x; g.gamma = L.g_in; g.w = L.wqkv; g.ws = L.sqkv; g.y = h->qkv; g.n = QKV; g.k = D;
        g.ts = ts_take(h, TL_K_QKV, gemv_fused_wavefronts(PRO_RMSNORM, EPI_DEQUANT, QKV, D));
        Prof p(h, TL_K_QKV, (double)QKV * D + QKV * 8.0 + D * 8.0);
        TL_LAUNCH(h, launch_gemv_fused(h->stream, PRO_RMSNORM, EPI_DEQUANT, g));
    }
    {
        Prof p(h, TL_K_ATTN, (double)c.n_heads * max_t * 128.0 + QKV * 4.0 + D * 4.0);
        unsigned long long* ts = ts_take(h, TL_K_ATTN, (int64_t)c.n_heads * 4);
        TL_LAUNCH(h, launch_attention_decode(h->stream, h->qkv, 1, c.n_heads, c.n_kv_heads, rowmap(h), h->rope_cos,
                                             h->rope_sin, h->kv, layer, h->kv_sk, h->kv_sv, h->att, max_t, ts));
    }
    {
        GemvArgs g = gemv_args(h);
        g.xf = h->att; g.w = L.wo; g.ws = L.so; g.residual = h->x; g.y = h->x; g.n = D; g.k = D;
        g.ts = ts_take(h, TL_K_O, gemv_fused_wavefronts(PRO_QUANT, EPI_DEQUANT_RES, D, D));
        Prof p(h, TL_K_O, (double)D * D + D * 4.0 + D * 12.0);
        TL_LAUNCH(h, launch_gemv_fused(h->stream, PRO_QUANT, EPI_DEQUANT_RES, g));
    }
    {
        GemvArgs g = gemv_args(h);
        g.xf = h->x; g.gamma = L.g_post; g.w = L.wg; g.w2 = L.wu; g.ws = L.sg; g.ws2 = L.su; g.y = h->hid;
        g.n = F; g.k = D;
        g.ts = ts_take(h, TL_K_GLU, gemv_fused_wavefronts(PRO_RMSNORM, EPI_GLU, F, D));
        Prof p(h, TL_K_GLU, 2.0 * F * D + F * 8.0 + D * 8.0 + F * 4.0);
        TL_LAUNCH(h, launch_gemv_fused(h->stream, PRO_RMSNORM, EPI_GLU, g));
    }
    {
        GemvArgs g = gemv_args(h);
        g.xf = h->hid; g.w = L.wd; g.ws = L.sd; g.residual = h->x; g.y = h->x; g.n = D; g.k = F;
        g.ts = ts_take(h, TL_K_DOWN, gemv_fused_wavefronts(PRO_QUANT, EPI_DEQUANT_RES, D, F));
        Prof p(h, TL_K_DOWN, (double)D * F + D * 4.0 + F * 4.0 + D * 8.0);
        TL_LAUNCH(h, launch_gemv_fused(h->stream, PRO_QUANT, EPI_DEQUANT_RES, g));
    }
    return TL_OK;
}

// K slice of a batched-decode GEMM: as many slices as keep the 32-column
// tiles times the slices within the 256 CUs (one round of 16-wavefront
// workgroups) and at least 16 chunks of 32 bytes (one per wavefront) in a
// slice.  At TinyLlama's shapes the down projection (64 tiles, K = 5632) is
// sliced in four and Q|K|V (80 tiles, K = 2048) in three: O and gate/up
// measured no faster sliced (the atomic adds and the fold cost what the
// spread gained; gate/up's 176 tiles leave no room for a second slice in one
// round)
static int32_t kslice_len(int32_t n, int32_t k) {
    const int tiles = n / 32, kch = k / 32;
    const int s = std::max(1, std::min(256 / std::max(tiles, 1), kch / 16));
    return ((kch + s - 1) / s) * 32;
}

// batched decode can run its down GEMM K-sliced
static bool kslice_ok(tl_handle* h, const LayerDev& L, int32_t rows) {
    const int D = h->D, F = h->F;
    return h->batch_kslice && rows > 1 && rows <= 32 && L.wd_p && D % 64 == 0 &&
           F % 64 == 0 && D <= 6144 && F <= 6144 && h->plan.n_leaves <= 64 && (size_t)rows * D <= h->racc_cap;
}

// batched decode can also run its Q|K|V GEMM K-sliced, its sums read by the
// grouped attention kernel
static bool qkv_kslice_ok(tl_handle* h, const LayerDev& L, int32_t rows, int32_t max_t) {
    const tl_config& c = h->cfg;
    return h->qkv_kslice && L.wqkv_p && h->QKV % 32 == 0 && (size_t)rows * h->QKV <= h->qacc_cap &&
           attention_decode_grouped(rows, c.n_heads, c.n_kv_heads, max_t);
}

// integer-sum GEMM into acc (h->racc or h->qacc, zero on entry; EPI_ACC),
// K-sliced; *clean is set false until the sums are consumed and cleared
static int32_t linear_acc(tl_handle* h, int32_t rows, const int8_t* wp, int32_t n, int32_t k, int kclass,
                          int32_t* acc, bool* clean) {
    GemmArgs a{};
    a.a = h->a8; a.as = h->as; a.wp = wp; a.acc = acc;
    a.m = rows; a.n = n; a.k = k; a.k_split = kslice_len(n, k);
    const double bytes = (double)rows * k + (double)n * k + (double)rows * n * 4.0;
    *clean = false;
    Prof p(h, kclass, bytes);
    TL_LAUNCH(h, launch_gemm_rows32(h->stream, EPI_ACC, a, rows32_waves(EPI_ACC)));
    return TL_OK;
}

// sums a failed batched step left in h->racc or h->qacc (between a K-sliced
// GEMM and the kernel that consumes and clears them): cleared before anything
// else uses the buffers
static int32_t discard_pending_sums(tl_handle* h) {
    if (!h->racc_clean || h->racc_res_ws) {
        TL_LAUNCH(h, launch_fill_u32(h->stream, (unsigned*)h->racc, (int32_t)h->racc_cap, 0u));
        h->racc_clean = true;
        h->racc_res_ws = nullptr;
    }
    if (!h->qacc_clean) {
        TL_LAUNCH(h, launch_fill_u32(h->stream, (unsigned*)h->qacc, (int32_t)h->qacc_cap, 0u));
        h->qacc_clean = true;
    }
    if (!h->qmax_clean) {
        TL_LAUNCH(h, launch_fill_u32(h->stream, h->qmax, kQmaxStride * h->max_rows, 0u));
        h->qmax_clean = true;
    }
    return TL_OK;
}

// prefill rows of this layer run their four GEMMs on packed operands: the
// row kernels then write h->a8 in the packed layout those GEMMs read
static bool prefill_packed(const tl_handle* h, const LayerDev& L, int32_t rows) {
    const int D = h->D, F = h->F, QKV = h->QKV;
    return rows >= 64 && L.wqkv_p && L.wo_p && L.wg_p && L.wu_p && L.wd_p &&
           D % 64 == 0 && F % 64 == 0 && D <= 6144 && F <= 6144 && h->plan.n_leaves <= 64 &&
           gemm_pk_supported(EPI_DEQUANT, rows, QKV, D) && gemm_pk_supported(EPI_DEQUANT_RES, rows, D, D) &&
           gemm_pk_supported(EPI_GLU, rows, F, D) && gemm_pk_supported(EPI_DEQUANT_RES, rows, D, F);
}

// RMSNorm + quantization of the rows of h->x into h->a8 / h->as (in the packed
// GEMM operand layout with pk), first adding a pending down projection's sums
// from h->racc (launch_rows_fold)
static int32_t rows_rmsnorm(tl_handle* h, int32_t rows, const float* g, bool pk = false,
                            const L2Prefetch* pf = nullptr) {
    if (h->racc_res_ws) {
        FoldArgs f{};
        f.x = h->x; f.acc = h->racc; f.as = h->as; f.ws = h->racc_res_ws; f.g = g;
        f.rows = rows; f.n = h->D; f.eps = h->cfg.rms_eps; f.plan = h->plan; f.q = h->a8; f.scales = h->as;
        if (pf) f.pf = *pf;
        h->racc_res_ws = nullptr;
        {
            Prof p(h, TL_K_NORM, (double)rows * h->D * 13.0);
            TL_LAUNCH(h, launch_rows_fold(h->stream, f));
        }
        h->racc_clean = true;
        return TL_OK;
    }
    Prof p(h, TL_K_NORM, (double)rows * h->D * 9.0);
    TL_LAUNCH(h, launch_rmsnorm_quant(h->stream, h->x, g, rows, h->D, h->cfg.rms_eps, h->plan, nullptr, h->a8, h->as,
                                      pk, pf));
    return TL_OK;
}

// one decoder layer (GI:256-281) for `rows` rows of h->x whose sequence and
// position are in h->row_seq / h->row_pos; max_t bounds pos + 1 over the rows.
// decode: every row is a different sequence (its own K/V row is appended by
// the attention kernel); otherwise the rows are consecutive prompt positions
// of one sequence (all appended before attention reads them).
int32_t layer_rows(tl_handle* h, int32_t layer, int32_t rows, int32_t max_t, bool decode) {
    if (rows == 1) return layer_row1(h, layer, max_t);
    const tl_config& c = h->cfg;
    const LayerDev& L = h->layers[layer];
    const int D = h->D, F = h->F, KVD = h->KVD, QKV = h->QKV;
    const bool ks = decode && kslice_ok(h, L, rows);
    const bool qks = ks && qkv_kslice_ok(h, L, rows, max_t);
    // the O GEMM K-sliced with the attention output quantized in it (one
    // 32-byte K chunk per wavefront of the 16-wavefront small-M GEMM)
    const bool of = qks && h->o_fuse && L.wo_p && c.n_heads <= 32 && c.n_heads % 4 == 0 &&
                    kslice_len(D, D) / 32 <= 16;
    const bool pk = !decode && prefill_packed(h, L, rows);   // h->a8 in the packed GEMM operand layout
    // prefill tiles on packed operands: qkv_post's work in the Q|K|V GEMM
    // epilogue, rotated Q in h->qkv ([rows][D]) quantized by the attention tiles
    const bool fq = pk && h->rows_one_seq && h->rows_pos0 + rows <= kTileMaxKeys && D % 64 == 0 &&
                    KVD % 64 == 0;
    // The row kernel before a GEMM also brings that GEMM's packed weight tiles
    // into the L2 of the XCD whose workgroups read them: the packed GEMMs'
    // grids have a multiple of 8 column tiles in x, so column tile t runs on
    // XCD t % 8 (batched decode: 32-column tiles; prefill: 64-column tiles,
    // gate/up's 32).  Batched decode prefetches for Q|K|V, gate/up and down
    // (O follows attention, not a row kernel); prefill for all four.
    auto pf_plan = [&](const int8_t* w0, const int8_t* w1, int nmat, int cols, int n, int k) {
        L2Prefetch p{};
        p.w[0] = w0;
        p.w[1] = w1;
        p.nmat = nmat;
        p.ntiles = n / cols;
        p.tile_bytes = (int64_t)cols * k;
        p.sink = h->pf_sink;
        return p;
    };
    const bool l2pf = ks || pk;
    const int tc = pk ? 64 : 32;
    const L2Prefetch pf_qkv = pf_plan(L.wqkv_p, nullptr, 1, tc, QKV, D), pf_o = pf_plan(L.wo_p, nullptr, 1, tc, D, D),
                     pf_glu = pf_plan(L.wg_p, L.wu_p, 2, 32, F, D), pf_down = pf_plan(L.wd_p, nullptr, 1, tc, D, F);
    const L2Prefetch* pfq = l2pf && (ks || fq) ? &pf_qkv : nullptr;   // prefill: the RoPE-epilogue tiles
    int32_t r;
    if (!ks && (r = discard_pending_sums(h))) return r;
    if ((r = rows_rmsnorm(h, rows, L.g_in, pk, pfq))) return r;
    if (qks) {
        // Q|K|V (K = D) K-sliced over the chip: the attention kernel
        // dequantizes the integer sums it reads from h->qacc
        if ((r = linear_acc(h, rows, L.wqkv_p, QKV, D, TL_K_QKV, h->qacc, &h->qacc_clean))) return r;
    } else if (fq) {
        GemmArgs a{};
        a.ap = h->a8; a.wp = L.wqkv_p; a.as = h->as; a.ws = L.sqkv; a.m = rows; a.n = QKV; a.k = D;
        const QkvRopeArgs f{h->rope_cos, h->rope_sin, rowmap(h), h->kv, layer, c.n_heads, c.n_kv_heads,
                            h->kv_sk, h->kv_sv, h->qkv, h->qmax};
        h->qmax_clean = false;
        Prof p(h, TL_K_QKV, (double)rows * D + (double)QKV * D + (double)rows * (D * 4.0 + KVD * 2.0));
        TL_LAUNCH(h, launch_gemm_pk_qkv(h->stream, a, f));
    } else if ((r = linear(h, EPI_DEQUANT, rows, h->a8, h->as, L.wqkv, L.sqkv, nullptr, nullptr, QKV, D, nullptr, h->qkv,
                           TL_K_QKV, L.wqkv_p, nullptr, pk))) {
        return r;
    }
    if (decode) {
        const QkvSums sums{h->qacc, h->as, L.sqkv};
        Prof p(h, TL_K_ATTN, (double)rows * c.n_kv_heads * (double)max_t * 128.0 + rows * QKV * 4.0);
        TL_LAUNCH(h, launch_attention_decode(h->stream, h->qkv, rows, c.n_heads, c.n_kv_heads, rowmap(h), h->rope_cos,
                                             h->rope_sin, h->kv, layer, h->kv_sk, h->kv_sv, h->att, max_t, nullptr,
                                             qks ? &sums : nullptr, of ? h->att_max : nullptr));
    } else if (fq) {
        Prof p(h, TL_K_ATTN, (double)rows * c.n_kv_heads * (double)max_t * 128.0 + rows * D * 8.0);
        TL_LAUNCH(h, launch_attention_tiles(h->stream, nullptr, nullptr, rows, c.n_heads, c.n_kv_heads, h->rows_seq,
                                            h->rows_pos0, h->kv, layer, h->kv_sk, h->kv_sv, h->att, h->qkv, h->qmax));
    } else {
        {
            Prof p(h, TL_K_ATTN, (double)rows * (QKV * 4.0 + D) + (double)rows * KVD * 2.0);
            TL_LAUNCH(h, launch_qkv_post(h->stream, h->qkv, rows, c.n_heads, c.n_kv_heads, rowmap(h), h->rope_cos,
                                         h->rope_sin, h->kv, layer, h->kv_sk, h->kv_sv, h->q8, h->qs, nullptr));
        }
        Prof p(h, TL_K_ATTN, (double)rows * c.n_kv_heads * (double)max_t * 128.0 + rows * D * 5.0);
        TL_LAUNCH(h, rows_attention(h, h->q8, h->qs, rows, layer, h->att, max_t));
    }
    if (of) {
        // the O GEMM K-sliced over the chip, quantizing the float32 attention
        // output itself at each row's maximum (from the heads' maxima); its
        // integer sums wait in h->racc for the post-attention RMSNorm, which
        // adds them to the residual and also clears the Q|K|V sums
        GemmArgs a{};
        a.a = h->a8; a.af = h->att; a.amax = h->att_max; a.amax_n = c.n_heads; a.as_out = h->as;
        a.wp = L.wo_p; a.acc = h->racc; a.m = rows; a.n = D; a.k = D; a.k_split = kslice_len(D, D);
        h->racc_clean = false;
        {
            Prof p(h, TL_K_O, (double)rows * D * 4.0 + (double)D * D + (double)rows * D * 4.0);
            TL_LAUNCH(h, launch_gemm_rows32(h->stream, EPI_ACC_F32, a, 16));
        }
        FoldArgs f{};
        f.x = h->x; f.acc = h->racc; f.as = h->as; f.ws = L.so; f.g = L.g_post;
        f.rows = rows; f.n = D; f.eps = c.rms_eps; f.plan = h->plan; f.q = h->a8; f.scales = h->as;
        f.zero = h->qacc; f.zero_n = QKV;
        if (l2pf) f.pf = pf_glu;
        {
            Prof p(h, TL_K_NORM, (double)rows * D * 13.0 + (double)rows * QKV * 4.0);
            TL_LAUNCH(h, launch_rows_fold(h->stream, f));
        }
        h->racc_clean = true;
        h->qacc_clean = true;
    } else {
        {
            // with the Q|K|V sums (or the Q row maxima) consumed, this kernel also
            // clears them
            int32_t* zero = qks ? h->qacc : (fq ? (int32_t*)h->qmax : nullptr);
            Prof p(h, TL_K_NORM, (double)rows * D * 5.0 + (qks ? (double)rows * QKV * 4.0 : 0.0));
            TL_LAUNCH(h, launch_quantize_rows(h->stream, h->att, rows, D, h->a8, h->as, zero,
                                              qks ? QKV : (fq ? kQmaxStride : 0), pk,
                                              l2pf && pk ? &pf_o : nullptr));
            if (qks) h->qacc_clean = true;
            if (fq) h->qmax_clean = true;
        }
        if ((r = linear(h, EPI_DEQUANT_RES, rows, h->a8, h->as, L.wo, L.so, nullptr, nullptr, D, D, h->x, h->x, TL_K_O,
                        L.wo_p, nullptr, pk)))
            return r;
        Prof p(h, TL_K_NORM, (double)rows * D * 9.0);
        TL_LAUNCH(h, launch_rmsnorm_quant(h->stream, h->x, L.g_post, rows, D, c.rms_eps, h->plan, nullptr, h->a8, h->as,
                                          pk, l2pf ? &pf_glu : nullptr));
    }
    if ((r = linear(h, EPI_GLU, rows, h->a8, h->as, L.wg, L.sg, L.wu, L.su, F, D, nullptr, h->hid, TL_K_GLU, L.wg_p,
                    L.wu_p, pk)))
        return r;
    {
        Prof p(h, TL_K_NORM, (double)rows * F * 5.0);
        TL_LAUNCH(h, launch_quantize_rows(h->stream, h->hid, rows, F, h->a8, h->as, nullptr, 0, pk,
                                          l2pf ? &pf_down : nullptr));
    }
    if (ks) {
        // the down GEMM (K = F) K-sliced over the chip: its integer sums wait
        // in h->racc for the next layer's input RMSNorm, or the final one
        if ((r = linear_acc(h, rows, L.wd_p, D, F, TL_K_DOWN, h->racc, &h->racc_clean))) return r;
        h->racc_res_ws = L.sd;
        return TL_OK;
    }
    if ((r = linear(h, EPI_DEQUANT_RES, rows, h->a8, h->as, L.wd, L.sd, nullptr, nullptr, D, F, h->x, h->x, TL_K_DOWN,
                    L.wd_p, nullptr, pk)))
        return r;
    return TL_OK;
}

// final RMSNorm + LM head + argmax for `rows` rows of h->x (row r predicts for
// sequence r when rows > 1, for `seq` when rows == 1), then record tokens
int32_t lm_head_rows(tl_handle* h, const float* xrow, int32_t rows, int32_t seq, int32_t advance) {
    const tl_config& c = h->cfg;
    const int D = h->D, V = c.vocab;
    unsigned long long* keys = h->keys + (rows == 1 ? seq : 0);
    int32_t n_wg = 0;   // rows == 1: the finalize kernel folds one key per LM-head workgroup
    EmbedNext nx{};     // rows == 1: and embeds the new token into row 0 for the next step
    if (rows == 1)
        nx = EmbedNext{h->emb, h->emb_s, h->D, c.vocab, h->x, h->row_pos, h->eos_id + seq, h->stopped + seq,
                       h->ctl_dev, h->ctl_dev + 1 + seq, nullptr};
    if (rows == 1) {
        GemvArgs g = gemv_args(h);
        g.xf = xrow; g.gamma = h->g_final; g.w = h->lm_w; g.ws = h->lm_s; g.key = keys; g.n = V; g.k = D;
        n_wg = gemv_fused_workgroups(PRO_RMSNORM, EPI_ARGMAX, V, D);
        if (n_wg <= 0 || n_wg > (V + 3) / 4) return fail(h, TL_ERR_INTERNAL, "LM head workgroup count");
        g.wg_keys = h->lm_wg_keys;
        g.ts = ts_take(h, TL_K_LMHEAD, gemv_fused_wavefronts(PRO_RMSNORM, EPI_ARGMAX, V, D));
        Prof p(h, TL_K_LMHEAD, (double)V * D + V * 4.0 + D * 8.0);
        TL_LAUNCH(h, launch_gemv_fused(h->stream, PRO_RMSNORM, EPI_ARGMAX, g));
    } else {
        if (h->racc_res_ws && xrow == h->x) {
            int32_t r = rows_rmsnorm(h, rows, h->g_final);
            if (r) return r;
        } else {
            int32_t r = discard_pending_sums(h);
            if (r) return r;
            Prof p(h, TL_K_NORM, (double)rows * D * 9.0);
            TL_LAUNCH(h, launch_rmsnorm_quant(h->stream, xrow, h->g_final, rows, D, c.rms_eps, h->plan, nullptr, h->a8, h->as));
        }
        GemmArgs a{};
        a.a = h->a8; a.w = h->lm_w; a.as = h->as; a.ws = h->lm_s; a.y = h->logits; a.m = rows; a.n = V; a.k = D;
        if (rows <= 32 && h->lm_wp && D % 64 == 0 && D <= 2048) {
            // packed-weight MFMA GEMM with the argmax in its epilogue (one key
            // per 32-column tile and row), then the tiles' keys folded per row
            const int tiles = V / 32;
            int32_t r = ensure_partials(h, (size_t)tiles * rows * 2);
            if (r) return r;
            a.wp = h->lm_wp;
            a.key = (unsigned long long*)h->partials;
            a.y = nullptr;
            Prof p(h, TL_K_LMHEAD, (double)V * D + V * 4.0 + (double)rows * D);
            TL_LAUNCH(h, launch_gemm_rows32(h->stream, EPI_ARGMAX, a, rows32_waves(EPI_ARGMAX)));
            TL_LAUNCH(h, launch_argmax_tiles(h->stream, a.key, tiles, rows, keys));
        } else {
            // MFMA GEMM writes logits, a row argmax folds them into keys
            int32_t r = run_gemm(h, EPI_DEQUANT, a, TL_K_LMHEAD);
            if (r) return r;
            TL_LAUNCH(h, launch_argmax_rows(h->stream, h->logits, rows, V, keys));
        }
    }
    if (rows == 1) nx.ts = ts_take(h, TL_K_OTHER, 1);
    TL_LAUNCH(h, launch_finalize_tokens(h->stream, keys, rows, h->token_cur + (rows == 1 ? seq : 0),
                                        h->tokens_out + (int64_t)(rows == 1 ? seq : 0) * c.max_pos, c.max_pos,
                                        h->n_gen + (rows == 1 ? seq : 0), h->cursor + (rows == 1 ? seq : 0),
                                        h->logit_out + (int64_t)(rows == 1 ? seq : 0) * c.max_pos, advance,
                                        h->lm_wg_keys, n_wg, nx));
    return TL_OK;
}

int32_t upload_rows(tl_handle* h, int32_t rows, int32_t seq_first, bool seq_per_row, int32_t pos0) {
    std::vector<int32_t> s(rows), p(rows);
    for (int i = 0; i < rows; i++) {
        s[i] = seq_per_row ? seq_first + i : seq_first;
        p[i] = pos0 + i;
    }
    h->rows_one_seq = !seq_per_row;
    h->rows_seq = seq_first;
    h->rows_pos0 = pos0;
    TL_HIP(h, hipMemcpyAsync(h->row_seq, s.data(), rows * sizeof(int32_t), hipMemcpyHostToDevice, h->stream));
    TL_HIP(h, hipMemcpyAsync(h->row_pos, p.data(), rows * sizeof(int32_t), hipMemcpyHostToDevice, h->stream));
    // the host vectors must outlive the async copies
    TL_HIP(h, hipStreamSynchronize(h->stream));
    return TL_OK;
}

// the EOS id a sequence's decode steps check, and its stop flag cleared
int32_t set_stop_state(tl_handle* h, int32_t seq, int32_t eos_id) {
    h->stop_state[0] = eos_id < 0 ? -1 : eos_id;
    h->stop_state[1] = 0;
    TL_HIP(h, hipMemcpyAsync(h->eos_id + seq, &h->stop_state[0], sizeof(int32_t), hipMemcpyHostToDevice, h->stream));
    TL_HIP(h, hipMemcpyAsync(h->stopped + seq, &h->stop_state[1], sizeof(int32_t), hipMemcpyHostToDevice, h->stream));
    // the host words must stay unchanged until the copies have run
    TL_HIP(h, hipStreamSynchronize(h->stream));
    return TL_OK;
}

// clears the abort word when a watched decode or prefill returns (also on an
// error path), so no later step of another call reads a stale abort
struct AbortWordReset {
    tl_handle* h;
    ~AbortWordReset() {
        if (h->ctl_host) *(volatile int32_t*)h->ctl_host = 0;
    }
};

int32_t check_model_loaded(tl_handle* h) {
    for (size_t l = 0; l < h->layers.size(); l++)
        if (!h->layers[l].wqkv) return fail(h, TL_ERR_BAD_DESCRIPTOR, "layer " + std::to_string(l) + " not loaded");
    return TL_OK;
}

// the embedding of row 0's sequence's current token at its cursor, before
// the first step of a decode call (later steps get it from the step before)
int32_t decode_embed1(tl_handle* h) {
    TL_LAUNCH(h, launch_embed_step(h->stream, h->token_cur, h->row_seq, 1, h->cursor, h->row_pos, h->D,
                                   h->cfg.vocab, h->emb, h->emb_s, h->x));
    return TL_OK;
}

// one batch-1 decode step of sequence seq (row 0 of the workspaces): 22
// fused layers over the embedding in row 0, fused LM head + argmax, then
// record the token, advance the cursor and embed the new token in row 0 at
// the new position for the next step.  Every argument is a fixed device
// pointer, so the step can be captured once and replayed.
int32_t decode_step1(tl_handle* h, int32_t seq, int32_t max_t) {
    const tl_config& c = h->cfg;
    int32_t r;
    for (int l = 0; l < c.n_layers; l++)
        if ((r = layer_row1(h, l, max_t))) return r;
    return lm_head_rows(h, h->x, 1, seq, 1);
}

int32_t decode_graph_launch(tl_handle* h, int32_t seq) {
    if ((int)h->graphs.size() < h->max_seqs) h->graphs.assign(h->max_seqs, nullptr);
    if (!h->graphs[seq]) {
        hipGraph_t g = nullptr;
        TL_HIP(h, hipStreamBeginCapture(h->stream, hipStreamCaptureModeThreadLocal));
        int32_t r = decode_step1(h, seq, h->cfg.max_pos);
        hipGraph_t cap = nullptr;
        hipError_t e = hipStreamEndCapture(h->stream, &cap);
        if (r) {
            if (cap) (void)hipGraphDestroy(cap);
            return r;
        }
        TL_HIP(h, e);
        g = cap;
        hipGraphExec_t ex = nullptr;
        e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        TL_HIP(h, e);
        h->graphs[seq] = ex;
    }
    TL_HIP(h, hipGraphLaunch(h->graphs[seq], h->stream));
    return TL_OK;
}

// one batched decode step of sequences 0..n_seqs-1 (rows r = sequence r):
// embed each sequence's current token at its cursor, the decoder layers at
// M = n_seqs, the LM head with its argmax, then record the tokens and advance
// the cursors.  Every argument is a fixed device pointer, so the step can be
// captured once per batch size and replayed.
int32_t batch_step(tl_handle* h, int32_t n_seqs, int32_t max_t) {
    const tl_config& c = h->cfg;
    int32_t r;
    if ((r = discard_pending_sums(h))) return r;
    TL_LAUNCH(h, launch_embed_step(h->stream, h->token_cur, h->row_seq, n_seqs, h->cursor, h->row_pos, h->D, c.vocab,
                                   h->emb, h->emb_s, h->x));
    for (int l = 0; l < c.n_layers; l++)
        if ((r = layer_rows(h, l, n_seqs, max_t, true))) return r;
    return lm_head_rows(h, h->x, n_seqs, 0, 1);
}

// replay of the captured batched step (captured on first use for this batch
// size, with the attention sized for the whole context)
int32_t batch_graph_launch(tl_handle* h, int32_t n_seqs) {
    if ((int)h->batch_graphs.size() <= h->max_seqs) h->batch_graphs.resize(h->max_seqs + 1, nullptr);
    if (!h->batch_graphs[n_seqs]) {
        TL_HIP(h, hipStreamBeginCapture(h->stream, hipStreamCaptureModeThreadLocal));
        int32_t r = batch_step(h, n_seqs, h->cfg.max_pos);
        hipGraph_t cap = nullptr;
        hipError_t e = hipStreamEndCapture(h->stream, &cap);
        if (r) {
            if (cap) (void)hipGraphDestroy(cap);
            return r;
        }
        TL_HIP(h, e);
        hipGraphExec_t ex = nullptr;
        e = hipGraphInstantiate(&ex, cap, nullptr, nullptr, 0);
        (void)hipGraphDestroy(cap);
        TL_HIP(h, e);
        h->batch_graphs[n_seqs] = ex;
    }
    TL_HIP(h, hipGraphLaunch(h->batch_graphs[n_seqs], h->stream));
    return TL_OK;
}

}  // namespace

// ===========================================================================
// C-ABI
// ===========================================================================
extern "C" {

const char* tl_status_string(int32_t s) {
    switch (s) {
        case TL_OK: return "ok";
        case TL_ERR_BAD_DESCRIPTOR: return "bad descriptor";
        case TL_ERR_UNSUPPORTED: return "unsupported";
        case TL_ERR_INTERNAL: return "internal error";
        default: return "unknown status";
    }
}

const char* tl_last_error(const tl_handle* h) { return h ? h->err.c_str() : g_create_error.c_str(); }

int32_t tl_create(const tl_config* cfg, int32_t max_seqs, tl_handle** out) {
    if (!cfg || !out) return fail(nullptr, TL_ERR_BAD_DESCRIPTOR, "null argument");
    *out = nullptr;
    const tl_config c = *cfg;
    if (c.head_dim != kHeadDim) return fail(nullptr, TL_ERR_UNSUPPORTED, "head_dim must be 64");
    if (c.hidden != c.n_heads * c.head_dim) return fail(nullptr, TL_ERR_BAD_DESCRIPTOR, "hidden != n_heads * head_dim");
    if (c.n_kv_heads < 1 || c.n_heads % c.n_kv_heads) return fail(nullptr, TL_ERR_BAD_DESCRIPTOR, "n_heads % n_kv_heads");
    if (c.n_heads / c.n_kv_heads > 8) return fail(nullptr, TL_ERR_UNSUPPORTED, "more than 8 query heads per KV head");
    if (c.hidden % 64 || c.intermediate % 64 || c.vocab % 64)
        return fail(nullptr, TL_ERR_UNSUPPORTED, "hidden, intermediate and vocab must be multiples of 64");
    if (c.hidden > 6144 || c.intermediate > 6144) return fail(nullptr, TL_ERR_UNSUPPORTED, "K above 6144");
    if (c.max_pos < 64 || c.max_pos % 64) return fail(nullptr, TL_ERR_UNSUPPORTED, "max_pos must be a multiple of 64");
    if (c.n_layers < 1 || max_seqs < 1) return fail(nullptr, TL_ERR_BAD_DESCRIPTOR, "n_layers and max_seqs must be >= 1");
    PwPlan plan;
    if (!make_pw_plan(c.hidden, &plan)) return fail(nullptr, TL_ERR_UNSUPPORTED, "hidden size has no perfect pairwise-sum tree");

    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) return fail(nullptr, TL_ERR_INTERNAL, "no HIP device");
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(nullptr, TL_ERR_INTERNAL, "hipGetDevice failed");
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return fail(nullptr, TL_ERR_INTERNAL, "hipGetDeviceProperties failed");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(nullptr, TL_ERR_UNSUPPORTED, std::string("kernels are built for gfx950, device is ") + prop.gcnArchName);

    tl_handle* h = new tl_handle();
    h->cfg = c;
    h->max_seqs = max_seqs;
    h->max_rows = std::max(c.max_pos, max_seqs);
    h->device = dev;
    h->plan = plan;
    h->D = c.hidden;
    h->F = c.intermediate;
    h->KVD = c.n_kv_heads * kHeadDim;
    h->QKV = h->D + 2 * h->KVD;
    h->layers.resize(c.n_layers);
    h->host_cursor.assign(max_seqs, 0);
    h->host_ngen.assign(max_seqs, 0);
    auto bad = [&](hipError_t e) {
        std::string m = std::string("allocation failed: ") + hipGetErrorString(e);
        tl_destroy(h);
        return fail(nullptr, TL_ERR_INTERNAL, m);
    };
    hipError_t e;
    if ((e = hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking)) != hipSuccess) return bad(e);
    const int R = h->max_rows, D = h->D, F = h->F;
    const int KF = std::max(D, F);
    if ((e = dalloc(h, &h->x, (size_t)R * D)) || (e = dalloc(h, &h->qkv, (size_t)R * h->QKV)) ||
        (e = dalloc(h, &h->a8, (size_t)((R + gemm_pk_row_pad() - 1) / gemm_pk_row_pad()) * gemm_pk_row_pad() * KF)) || (e = dalloc(h, &h->as, (size_t)R)) ||
        (e = dalloc(h, &h->q8, (size_t)R * D)) || (e = dalloc(h, &h->qs, (size_t)R)) ||
        (e = dalloc(h, &h->att, (size_t)R * D)) || (e = dalloc(h, &h->hid, (size_t)R * F)) ||
        (e = dalloc(h, &h->logits, (size_t)max_seqs * c.vocab)) || (e = dalloc(h, &h->row_seq, (size_t)R)) || (e = dalloc(h, &h->tile_ctr, (size_t)kSkinnyTiles)) ||
        (e = dalloc(h, &h->row_pos, (size_t)R)) || (e = dalloc(h, &h->tokens, (size_t)R)) ||
        (e = dalloc(h, &h->fscratch, 64)) || (e = dalloc(h, &h->op_key, 1)) || (e = dalloc(h, &h->keys, (size_t)max_seqs)) ||
        (e = dalloc(h, &h->lm_wg_keys, (size_t)(c.vocab + 3) / 4)) ||
        (e = dalloc(h, &h->token_cur, (size_t)max_seqs)) || (e = dalloc(h, &h->cursor, (size_t)max_seqs)) ||
        (e = dalloc(h, &h->n_gen, (size_t)max_seqs)) || (e = dalloc(h, &h->eos_id, (size_t)max_seqs)) ||
        (e = dalloc(h, &h->stopped, (size_t)max_seqs)) ||
        (e = dalloc(h, &h->racc, h->racc_cap = (size_t)std::min(32, max_seqs) * D)) ||
        (e = dalloc(h, &h->qacc, h->qacc_cap = (size_t)std::min(32, max_seqs) * h->QKV)) ||
        (e = dalloc(h, &h->pf_sink, 1)) ||
        (e = dalloc(h, &h->qmax, (size_t)kQmaxStride * R)) ||
        (e = dalloc(h, &h->tokens_out, (size_t)max_seqs * c.max_pos)) ||
        (e = dalloc(h, &h->logit_out, (size_t)max_seqs * c.max_pos)) ||
        (e = dalloc(h, &h->rope_cos, (size_t)c.max_pos * kHeadDim)) || (e = dalloc(h, &h->att_max, (size_t)R * c.n_heads)) ||
        (e = dalloc(h, &h->rope_sin, (size_t)c.max_pos * kHeadDim)) ||
        (e = dalloc(h, &h->kv_sk, (size_t)c.n_layers * c.n_kv_heads)) ||
        (e = dalloc(h, &h->kv_sv, (size_t)c.n_layers * c.n_kv_heads)) ||
        (e = dalloc(h, &h->g_final, (size_t)D)) || (e = dalloc(h, &h->lm_w, (size_t)c.vocab * D)) ||
        (e = dalloc(h, &h->lm_s, (size_t)c.vocab)) || (e = dalloc(h, &h->emb, (size_t)c.vocab * D)) ||
        (e = dalloc(h, &h->emb_s, (size_t)c.vocab)) ||
        (e = dalloc(h, &h->kv_stage, (size_t)2 * c.max_pos * kHeadDim)))
        return bad(e);
    const size_t plane = (size_t)c.max_pos * kHeadDim;
    const size_t kv_bytes = (size_t)max_seqs * c.n_layers * c.n_kv_heads * plane;
    if ((e = dalloc(h, &h->kv.k, kv_bytes)) || (e = dalloc(h, &h->kv.v, kv_bytes))) return bad(e);
    h->kv.n_layers = c.n_layers;
    h->kv.n_kv_heads = c.n_kv_heads;
    h->kv.max_pos = c.max_pos;
    if ((e = hipMemsetAsync(h->kv.k, 0, kv_bytes, h->stream)) || (e = hipMemsetAsync(h->kv.v, 0, kv_bytes, h->stream)) ||
        (e = hipMemsetAsync(h->keys, 0, sizeof(unsigned long long) * max_seqs, h->stream)) ||
        (e = hipMemsetAsync(h->cursor, 0, sizeof(int32_t) * max_seqs, h->stream)) ||
        (e = hipMemsetAsync(h->n_gen, 0, sizeof(int32_t) * max_seqs, h->stream)) ||
        (e = hipMemsetAsync(h->eos_id, 0xFF, sizeof(int32_t) * max_seqs, h->stream)) ||
        (e = hipMemsetAsync(h->stopped, 0, sizeof(int32_t) * max_seqs, h->stream)) ||
        (e = hipMemsetAsync(h->tile_ctr, 0, sizeof(unsigned) * kSkinnyTiles, h->stream)) ||
        (e = hipMemsetAsync(h->racc, 0, sizeof(int32_t) * h->racc_cap, h->stream)) ||
        (e = hipMemsetAsync(h->qacc, 0, sizeof(int32_t) * h->qacc_cap, h->stream)) ||
        (e = hipMemsetAsync(h->qmax, 0, sizeof(unsigned) * kQmaxStride * R, h->stream)))
        return bad(e);
    std::vector<float> cs, sn;
    default_rope(c.max_pos, c.rope_theta, cs, sn);
    if ((e = hipMemcpy(h->rope_cos, cs.data(), cs.size() * sizeof(float), hipMemcpyHostToDevice)) ||
        (e = hipMemcpy(h->rope_sin, sn.data(), sn.size() * sizeof(float), hipMemcpyHostToDevice)))
        return bad(e);
    h->rope_n = c.max_pos;
    {
        void* sp = nullptr;
        if ((e = scratch_address(dev, &sp, &h->noalloc_done))) return bad(e);
        h->noalloc_scratch = (int32_t*)sp;
    }
    {
        // the abort word and the stop mirrors: pinned, coherent host memory
        // that the token bookkeeping kernel reads and writes every step
        void* hp = nullptr;
        void* dp = nullptr;
        const size_t words = 1 + (size_t)max_seqs;
        if ((e = hipHostMalloc(&hp, sizeof(int32_t) * words, hipHostMallocMapped | hipHostMallocCoherent))) return bad(e);
        h->ctl_host = (int32_t*)hp;
        std::memset(hp, 0, sizeof(int32_t) * words);
        if ((e = hipHostGetDevicePointer(&dp, hp, 0))) return bad(e);
        h->ctl_dev = (int32_t*)dp;
        for (auto& ev : h->watch_ev)
            if ((e = hipEventCreateWithFlags(&ev, hipEventDisableTiming))) return bad(e);
    }
    if ((e = init_kernels())) return bad(e);
    if ((e = init_decode_kernels())) return bad(e);
    if ((e = init_prefill_kernels())) return bad(e);
    if ((e = init_gemm_pk_kernels())) return bad(e);
    if ((e = init_skinny_kernels())) return bad(e);
    if (const char* env = std::getenv("TL_BATCH_O_FUSE")) h->o_fuse = env[0] != '0';
    if (const char* env = std::getenv("TL_BATCH_KSLICE")) h->batch_kslice = env[0] != '0';
    if (const char* env = std::getenv("TL_BATCH_QKV_KSLICE")) h->qkv_kslice = env[0] != '0';
    if ((e = hipStreamSynchronize(h->stream))) return bad(e);
    *out = h;
    return TL_OK;
}

void tl_destroy(tl_handle* h) {
    if (!h) return;
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    for (auto& p : h->prof_pending) {
        (void)hipEventDestroy(p.start);
        (void)hipEventDestroy(p.stop);
    }
    for (auto e : h->event_pool) (void)hipEventDestroy(e);
    for (auto g : h->graphs)
        if (g) (void)hipGraphExecDestroy(g);
    for (auto g : h->batch_graphs)
        if (g) (void)hipGraphExecDestroy(g);
    for (void* p : h->allocs) (void)hipFree(p);
    for (auto e : h->watch_ev)
        if (e) (void)hipEventDestroy(e);
    if (h->ctl_host) (void)hipHostFree(h->ctl_host);
    if (h->stream) (void)hipStreamDestroy(h->stream);
    delete h;
}

int32_t tl_get_config(const tl_handle* h, tl_config* cfg) {
    if (!h || !cfg) return TL_ERR_BAD_DESCRIPTOR;
    *cfg = h->cfg;
    return TL_OK;
}

int32_t tl_sync(tl_handle* h) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    return finish(h);
}

int32_t tl_load_layer(tl_handle* h, int32_t layer, const int8_t* const w[7], const float* const s[7],
                      const float* g_in, const float* g_post, int32_t src) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, layer >= 0 && layer < h->cfg.n_layers, "layer out of range");
    TL_REQ(h, w && s && g_in && g_post, "null weight pointer");
    for (int i = 0; i < 7; i++) TL_REQ(h, w[i] && s[i], "null weight pointer");
    LayerDev& L = h->layers[layer];
    const int D = h->D, F = h->F, KVD = h->KVD;
    if (!L.wqkv) {
        TL_HIP(h, dalloc(h, &L.wqkv, (size_t)h->QKV * D));
        TL_HIP(h, dalloc(h, &L.sqkv, (size_t)h->QKV));
        TL_HIP(h, dalloc(h, &L.wo, (size_t)D * D));
        TL_HIP(h, dalloc(h, &L.so, (size_t)D));
        TL_HIP(h, dalloc(h, &L.wg, (size_t)F * D));
        TL_HIP(h, dalloc(h, &L.sg, (size_t)F));
        TL_HIP(h, dalloc(h, &L.wu, (size_t)F * D));
        TL_HIP(h, dalloc(h, &L.su, (size_t)F));
        TL_HIP(h, dalloc(h, &L.wd, (size_t)D * F));
        TL_HIP(h, dalloc(h, &L.sd, (size_t)D));
        TL_HIP(h, dalloc(h, &L.g_in, (size_t)D));
        TL_HIP(h, dalloc(h, &L.g_post, (size_t)D));
    }
    TL_HIP(h, copy_in(h, L.wqkv, w[0], (size_t)D * D, src));
    TL_HIP(h, copy_in(h, L.wqkv + (size_t)D * D, w[1], (size_t)KVD * D, src));
    TL_HIP(h, copy_in(h, L.wqkv + (size_t)(D + KVD) * D, w[2], (size_t)KVD * D, src));
    TL_HIP(h, copy_in(h, L.sqkv, s[0], sizeof(float) * D, src));
    TL_HIP(h, copy_in(h, L.sqkv + D, s[1], sizeof(float) * KVD, src));
    TL_HIP(h, copy_in(h, L.sqkv + D + KVD, s[2], sizeof(float) * KVD, src));
    TL_HIP(h, copy_in(h, L.wo, w[3], (size_t)D * D, src));
    TL_HIP(h, copy_in(h, L.so, s[3], sizeof(float) * D, src));
    TL_HIP(h, copy_in(h, L.wg, w[4], (size_t)F * D, src));
    TL_HIP(h, copy_in(h, L.sg, s[4], sizeof(float) * F, src));
    TL_HIP(h, copy_in(h, L.wu, w[5], (size_t)F * D, src));
    TL_HIP(h, copy_in(h, L.su, s[5], sizeof(float) * F, src));
    TL_HIP(h, copy_in(h, L.wd, w[6], (size_t)D * F, src));
    TL_HIP(h, copy_in(h, L.sd, s[6], sizeof(float) * D, src));
    TL_HIP(h, copy_in(h, L.g_in, g_in, sizeof(float) * D, src));
    TL_HIP(h, copy_in(h, L.g_post, g_post, sizeof(float) * D, src));
    if (D % 32 == 0 && F % 32 == 0 && KVD % 32 == 0) {
        if (!L.wqkv_p) {
            TL_HIP(h, dalloc(h, &L.wqkv_p, (size_t)h->QKV * D));
            TL_HIP(h, dalloc(h, &L.wo_p, (size_t)D * D));
            TL_HIP(h, dalloc(h, &L.wg_p, (size_t)F * D));
            TL_HIP(h, dalloc(h, &L.wu_p, (size_t)F * D));
            TL_HIP(h, dalloc(h, &L.wd_p, (size_t)D * F));
        }
        TL_LAUNCH(h, launch_pack_weights(h->stream, L.wqkv, h->QKV, D, L.wqkv_p));
        TL_LAUNCH(h, launch_pack_weights(h->stream, L.wo, D, D, L.wo_p));
        TL_LAUNCH(h, launch_pack_weights(h->stream, L.wg, F, D, L.wg_p));
        TL_LAUNCH(h, launch_pack_weights(h->stream, L.wu, F, D, L.wu_p));
        TL_LAUNCH(h, launch_pack_weights(h->stream, L.wd, D, F, L.wd_p));
    }
    return finish(h);
}

int32_t tl_load_lm_head(tl_handle* h, const int8_t* w, const float* s, const float* g_final, int32_t src) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, w && s && g_final, "null pointer");
    TL_HIP(h, copy_in(h, h->lm_w, w, (size_t)h->cfg.vocab * h->D, src));
    TL_HIP(h, copy_in(h, h->lm_s, s, sizeof(float) * h->cfg.vocab, src));
    TL_HIP(h, copy_in(h, h->g_final, g_final, sizeof(float) * h->D, src));
    if (h->cfg.vocab % 32 == 0 && h->D % 32 == 0) {
        if (!h->lm_wp) TL_HIP(h, dalloc(h, &h->lm_wp, (size_t)h->cfg.vocab * h->D));
        TL_LAUNCH(h, launch_pack_weights(h->stream, h->lm_w, h->cfg.vocab, h->D, h->lm_wp));
    }
    return finish(h);
}

int32_t tl_load_embedding(tl_handle* h, const int8_t* e, const float* s, int32_t src) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, e && s, "null pointer");
    TL_HIP(h, copy_in(h, h->emb, e, (size_t)h->cfg.vocab * h->D, src));
    TL_HIP(h, copy_in(h, h->emb_s, s, sizeof(float) * h->cfg.vocab, src));
    return finish(h);
}

int32_t tl_set_kv_scales(tl_handle* h, const float* k_scales, const float* v_scales) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, k_scales && v_scales, "null pointer");
    const size_t n = (size_t)h->cfg.n_layers * h->cfg.n_kv_heads;
    for (size_t i = 0; i < n; i++)
        TL_REQ(h, k_scales[i] > 0.0f && v_scales[i] > 0.0f && std::isfinite(k_scales[i]) && std::isfinite(v_scales[i]),
               "KV scales must be positive and finite");
    TL_HIP(h, hipMemcpyAsync(h->kv_sk, k_scales, n * sizeof(float), hipMemcpyHostToDevice, h->stream));
    TL_HIP(h, hipMemcpyAsync(h->kv_sv, v_scales, n * sizeof(float), hipMemcpyHostToDevice, h->stream));
    return finish(h);
}

int32_t tl_set_rope_table(tl_handle* h, const float* cos, const float* sin, int32_t n_pos) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, cos && sin, "null pointer");
    TL_REQ(h, n_pos >= h->cfg.max_pos, "RoPE table shorter than max_pos");
    const size_t n = (size_t)h->cfg.max_pos * kHeadDim * sizeof(float);
    TL_HIP(h, hipMemcpyAsync(h->rope_cos, cos, n, hipMemcpyHostToDevice, h->stream));
    TL_HIP(h, hipMemcpyAsync(h->rope_sin, sin, n, hipMemcpyHostToDevice, h->stream));
    return finish(h);
}

int32_t tl_kv_write(tl_handle* h, int32_t seq, int32_t layer, int32_t g, int32_t t0, int32_t n,
                    const int8_t* k_rows, const int8_t* v_rows) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    const tl_config& c = h->cfg;
    TL_REQ(h, seq >= 0 && seq < h->max_seqs && layer >= 0 && layer < c.n_layers && g >= 0 && g < c.n_kv_heads,
           "KV index out of range");
    TL_REQ(h, t0 >= 0 && n >= 0 && (int64_t)t0 + n <= c.max_pos, "KV token range out of bounds");
    if (n == 0) return TL_OK;
    // rows pass through the handle's staging buffer (n <= max_pos rows each)
    const size_t bytes = (size_t)n * kHeadDim;
    int8_t* kd = h->kv_stage;
    int8_t* vd = h->kv_stage + (size_t)c.max_pos * kHeadDim;
    if (k_rows) TL_HIP(h, hipMemcpyAsync(kd, k_rows, bytes, hipMemcpyHostToDevice, h->stream));
    if (v_rows) TL_HIP(h, hipMemcpyAsync(vd, v_rows, bytes, hipMemcpyHostToDevice, h->stream));
    TL_LAUNCH(h, launch_kv_scatter(h->stream, h->kv, seq, layer, g, t0, n, k_rows ? kd : nullptr, v_rows ? vd : nullptr));
    return finish(h);
}

int32_t tl_kv_read(tl_handle* h, int32_t seq, int32_t layer, int32_t g, int32_t t0, int32_t n,
                   int8_t* k_rows, int8_t* v_rows) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    const tl_config& c = h->cfg;
    TL_REQ(h, seq >= 0 && seq < h->max_seqs && layer >= 0 && layer < c.n_layers && g >= 0 && g < c.n_kv_heads,
           "KV index out of range");
    TL_REQ(h, t0 >= 0 && n >= 0 && (int64_t)t0 + n <= c.max_pos, "KV token range out of bounds");
    if (n == 0) return TL_OK;
    const size_t bytes = (size_t)n * kHeadDim;
    int8_t* kd = h->kv_stage;
    int8_t* vd = h->kv_stage + (size_t)c.max_pos * kHeadDim;
    TL_LAUNCH(h, launch_kv_gather(h->stream, h->kv, seq, layer, g, t0, n, kd, vd));
    if (k_rows) TL_HIP(h, hipMemcpyAsync(k_rows, kd, bytes, hipMemcpyDeviceToHost, h->stream));
    if (v_rows) TL_HIP(h, hipMemcpyAsync(v_rows, vd, bytes, hipMemcpyDeviceToHost, h->stream));
    return finish(h);
}

// ---- operators ----------------------------------------------------------------

int32_t tl_quantize_rows(tl_handle* h, const float* x, int32_t rows, int32_t n, int8_t* q, double* scales) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, rows >= 0 && n > 0 && x && q && scales, "bad quantize_rows arguments");
    TL_LAUNCH(h, launch_quantize_rows(h->stream, x, rows, n, q, scales));
    return finish(h);
}

int32_t tl_quantize_tensor(tl_handle* h, const float* x, int64_t n, int8_t* q, double* scale) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, n >= 0 && x && q && scale, "bad quantize_tensor arguments");
    TL_LAUNCH(h, launch_quantize_tensor(h->stream, x, n, q, scale, h->fscratch));
    return finish(h);
}

int32_t tl_quantize_weight_rows(tl_handle* h, const float* w, int32_t rows, int32_t n, int8_t* q, float* scales) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, rows >= 0 && n > 0 && w && q && scales, "bad quantize_weight_rows arguments");
    TL_LAUNCH(h, launch_quantize_weight_rows(h->stream, w, rows, n, q, scales));
    return finish(h);
}

int32_t tl_rmsnorm_quant(tl_handle* h, const float* x, const float* gamma, int32_t rows, int32_t n, float* y,
                         int8_t* q, double* scales) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, rows >= 0 && x && gamma && q && scales, "bad rmsnorm arguments");
    PwPlan plan;
    if (!make_pw_plan(n, &plan)) return fail(h, TL_ERR_UNSUPPORTED, "width has no perfect pairwise-sum tree");
    TL_LAUNCH(h, launch_rmsnorm_quant(h->stream, x, gamma, rows, n, h->cfg.rms_eps, plan, y, q, scales));
    return finish(h);
}

int32_t tl_gemv_i8_requant(tl_handle* h, const int8_t* x, const int8_t* w, const float* m, int32_t n, int32_t k,
                           int8_t* y, int32_t* acc) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, x && w && m && y && n > 0, "bad gemv arguments");
    TL_REQ(h, k > 0 && k % 16 == 0 && k <= 6144, "K must be a positive multiple of 16, at most 6144");
    GemvArgs g{};
    g.w = w; g.ws = m; g.x = x; g.y8 = y; g.acc = acc; g.n = n; g.k = k;
    {
        Prof p(h, TL_K_QKV, (double)n * k + n * 4.0 + k + n);
        TL_LAUNCH(h, launch_gemv(h->stream, EPI_REQUANT, g));
    }
    return finish(h);
}

int32_t tl_requant_q16(tl_handle* h, const int32_t* acc, const uint32_t* scale_q16, int32_t n, int32_t active,
                       int32_t lanes_per_scale, int32_t nonnegative_only, int8_t* y) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, acc && scale_q16 && y && n >= 0, "bad requantize arguments");
    TL_REQ(h, lanes_per_scale >= 1, "lanes_per_scale must be at least 1");
    TL_REQ(h, active >= 0 && active <= n, "active lane count outside 0..n");
    TL_LAUNCH(h, launch_requant_q16(h->stream, acc, scale_q16, n, active, lanes_per_scale, nonnegative_only != 0, y));
    return finish(h);
}

int32_t tl_causal_mask_i32(tl_handle* h, const int32_t* scores, int32_t rows, int32_t cols, int32_t query_pos_base,
                           int32_t key_pos_base, int32_t query_row_count, int32_t key_col_count, int32_t* out) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, scores && out && rows >= 0 && cols > 0, "bad causal mask arguments");
    TL_REQ(h, query_pos_base >= 0 && key_pos_base >= 0 && query_row_count >= 0 && key_col_count >= 0,
           "negative position or count");
    TL_LAUNCH(h, launch_causal_mask_i32(h->stream, scores, rows, cols, query_pos_base, key_pos_base, query_row_count,
                                        key_col_count, out));
    return finish(h);
}

int32_t tl_rope_q16(tl_handle* h, const int8_t* x, int32_t rows, int32_t n_heads, const int32_t* pos, int8_t* out) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, x && pos && out && rows >= 0 && n_heads > 0, "bad rope arguments");
    std::vector<int32_t> hp(rows);
    if (rows > 0) TL_HIP(h, hipMemcpy(hp.data(), pos, sizeof(int32_t) * rows, hipMemcpyDefault));
    for (int32_t r = 0; r < rows; r++)
        TL_REQ(h, hp[r] >= 0 && hp[r] < h->rope_n, "position outside the RoPE table");
    TL_LAUNCH(h, launch_rope_q16(h->stream, x, rows, n_heads, pos, h->rope_cos, h->rope_sin, h->rope_n, out));
    return finish(h);
}

int32_t tl_argmax_i32(tl_handle* h, const int32_t* v, int32_t n, int32_t* index, int32_t* value) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, v && index && n > 0, "bad argmax arguments");
    TL_LAUNCH(h, launch_argmax_i32(h->stream, v, n, h->op_key));
    unsigned long long key = 0;
    TL_HIP(h, hipMemcpyAsync(&key, h->op_key, sizeof key, hipMemcpyDeviceToHost, h->stream));
    int32_t r = finish(h);
    if (r) return r;
    *index = (int32_t)(0xFFFFFFFFu - (unsigned)(key & 0xFFFFFFFFull));
    if (value) *value = (int32_t)((unsigned)(key >> 32) ^ 0x80000000u);
    return TL_OK;
}

int32_t tl_gemm_i8(tl_handle* h, const int8_t* a, const int8_t* w, int32_t m, int32_t n, int32_t k, int32_t* c) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, a && w && c && m > 0 && n > 0, "bad gemm arguments");
    TL_REQ(h, k > 0 && k % 64 == 0, "K must be a positive multiple of 64");
    GemmArgs g{};
    g.a = a; g.w = w; g.acc = c; g.m = m; g.n = n; g.k = k;
    int32_t r = run_gemm(h, EPI_RAW, g, TL_K_GEMM_PREFILL);
    if (r) return r;
    return finish(h);
}

int32_t tl_gemm_i8_noalloc(tl_handle* h, const int8_t* a, const int8_t* w, int32_t m, int32_t n, int32_t k,
                           int32_t* c) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, a && w && c && m > 0 && n > 0, "bad gemm arguments");
    TL_REQ(h, k > 0 && k % 64 == 0, "K must be a positive multiple of 64");
    TL_REQ(h, h->noalloc_scratch, "no fixed scratch on this device");
    GemmArgs g{};
    g.a = a; g.w = w; g.acc = c; g.m = m; g.n = n; g.k = k;
    const FixedScratch fx{h->noalloc_scratch, kNoAllocPartials, (unsigned*)(h->noalloc_scratch + kNoAllocPartials),
                          kNoAllocCounters};
    {
        // after the previous user of this GPU's array, from any handle
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        TL_HIP(h, hipStreamWaitEvent(h->stream, h->noalloc_done, 0));
        const int32_t r = run_gemm(h, EPI_RAW, g, TL_K_GEMM_PREFILL, &fx);
        const hipError_t e = hipEventRecord(h->noalloc_done, h->stream);
        if (r) return r;
        TL_HIP(h, e);
    }
    return finish(h);
}

int32_t tl_gemm_i8_dequant(tl_handle* h, const int8_t* a, const double* a_scales, const int8_t* w,
                           const float* w_scales, int32_t m, int32_t n, int32_t k, const float* residual, float* y) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, a && a_scales && w && w_scales && y && m > 0 && n > 0, "bad gemm arguments");
    if (m == 1) TL_REQ(h, k > 0 && k % 16 == 0 && k <= 6144, "K must be a multiple of 16, at most 6144");
    else TL_REQ(h, k > 0 && k % 64 == 0, "K must be a positive multiple of 64");
    int32_t r = linear(h, residual ? EPI_DEQUANT_RES : EPI_DEQUANT, m, a, a_scales, w, w_scales, nullptr, nullptr, n, k,
                       residual, y, TL_K_OTHER);
    if (r) return r;
    return finish(h);
}

int32_t tl_rope(tl_handle* h, float* v, int32_t rows, int32_t n_heads, const int32_t* pos) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, v && pos && rows >= 0 && n_heads > 0, "bad rope arguments");
    TL_LAUNCH(h, launch_rope(h->stream, v, rows, n_heads, pos, h->rope_cos, h->rope_sin));
    return finish(h);
}

int32_t tl_linear_f32(tl_handle* h, const float* x, const float* w, const float* b, const float* residual, int32_t m,
                      int32_t n, int32_t k, float* y) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, x && w && y && m >= 0 && n >= 0 && k >= 0, "bad linear arguments");
    TL_LAUNCH(h, launch_linear_f32(h->stream, x, w, b, residual, m, n, k, y));
    return finish(h);
}

int32_t tl_attention_f32(tl_handle* h, const float* q, const float* k, const float* v, int32_t seq, int32_t n_heads,
                         int32_t n_kv_heads, float scale, float* out, float* scores, float* weights) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, q && k && v && out, "null pointer");
    TL_REQ(h, seq >= 0 && seq <= kTileMaxKeys, "sequence longer than 4096 tokens");
    TL_REQ(h, n_heads >= 1 && n_kv_heads >= 1 && n_heads % n_kv_heads == 0, "heads must be a multiple of KV heads");
    TL_LAUNCH(h, launch_attention_f32(h->stream, q, k, v, seq, n_heads, n_kv_heads, scale, out, scores, weights));
    return finish(h);
}

int32_t tl_softmax_rows(tl_handle* h, const float* x, int32_t rows, int32_t n, float* p) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, x && p && rows >= 0 && n > 0, "bad softmax arguments");
    TL_LAUNCH(h, launch_softmax_rows(h->stream, x, rows, n, p));
    return finish(h);
}

int32_t tl_silu_mul(tl_handle* h, const float* g, const float* u, int64_t n, float* y) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, g && y && n >= 0, "bad silu arguments");
    TL_LAUNCH(h, launch_silu_mul(h->stream, g, u, n, y));
    return finish(h);
}

int32_t tl_qkv_append(tl_handle* h, int32_t seq, int32_t layer, int32_t pos0, int32_t rows, const float* qkv,
                      int8_t* q8, double* q_scale, float* q_rot) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    const tl_config& c = h->cfg;
    TL_REQ(h, seq >= 0 && seq < h->max_seqs && layer >= 0 && layer < c.n_layers, "index out of range");
    TL_REQ(h, rows >= 1 && rows <= h->max_rows && pos0 >= 0 && (int64_t)pos0 + rows <= c.max_pos,
           "position range out of bounds");
    TL_REQ(h, qkv && q8 && q_scale, "null pointer");
    int32_t r = upload_rows(h, rows, seq, false, pos0);
    if (r) return r;
    TL_LAUNCH(h, launch_qkv_post(h->stream, qkv, rows, c.n_heads, c.n_kv_heads, rowmap(h), h->rope_cos, h->rope_sin,
                                 h->kv, layer, h->kv_sk, h->kv_sv, q8, q_scale, q_rot));
    return finish(h);
}

int32_t tl_attention(tl_handle* h, int32_t seq, int32_t layer, int32_t pos0, int32_t rows, const int8_t* q8,
                     const double* q_scale, float* out) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    const tl_config& c = h->cfg;
    TL_REQ(h, seq >= 0 && seq < h->max_seqs && layer >= 0 && layer < c.n_layers, "index out of range");
    TL_REQ(h, rows >= 1 && rows <= h->max_rows && pos0 >= 0 && (int64_t)pos0 + rows <= c.max_pos,
           "position range out of bounds");
    TL_REQ(h, q8 && q_scale && out, "null pointer");
    int32_t r = upload_rows(h, rows, seq, false, pos0);
    if (r) return r;
    {
        Prof p(h, TL_K_ATTN, 0.0);
        TL_LAUNCH(h, rows_attention(h, q8, q_scale, rows, layer, out, pos0 + rows));
    }
    return finish(h);
}

int32_t tl_lm_head_argmax(tl_handle* h, const float* x, int32_t* token, float* logit, float* logits) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, x && token, "null pointer");
    const int D = h->D, V = h->cfg.vocab;
    TL_LAUNCH(h, launch_reset_keys(h->stream, h->op_key, 1));
    {
        Prof p(h, TL_K_NORM, D * 9.0);
        TL_LAUNCH(h, launch_rmsnorm_quant(h->stream, x, h->g_final, 1, D, h->cfg.rms_eps, h->plan, nullptr, h->a8, h->as));
    }
    GemvArgs g{};
    g.w = h->lm_w; g.ws = h->lm_s; g.x = h->a8; g.xs = h->as; g.key = h->op_key; g.y = logits; g.n = V; g.k = D;
    {
        Prof p(h, TL_K_LMHEAD, (double)V * D + V * 4.0 + D);
        TL_LAUNCH(h, launch_gemv(h->stream, EPI_ARGMAX, g));
    }
    unsigned long long key = 0;
    TL_HIP(h, hipMemcpyAsync(&key, h->op_key, sizeof key, hipMemcpyDeviceToHost, h->stream));
    int32_t r = finish(h);
    if (r) return r;
    *token = (int32_t)(0xFFFFFFFFu - (unsigned)(key & 0xFFFFFFFFull));
    if (logit) {
        unsigned u = (unsigned)(key >> 32);
        u = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
        std::memcpy(logit, &u, sizeof u);
    }
    return TL_OK;
}

// ---- composed path ----------------------------------------------------------------

int32_t tl_embed(tl_handle* h, const int32_t* tokens, int32_t rows, float* x) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, tokens && x && rows >= 0, "bad embed arguments");
    TL_LAUNCH(h, launch_embed(h->stream, tokens, rows, h->D, h->cfg.vocab, h->emb, h->emb_s, x));
    return finish(h);
}

int32_t tl_decode_layer(tl_handle* h, int32_t seq, int32_t layer, int32_t pos, float* x) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    const tl_config& c = h->cfg;
    TL_REQ(h, seq >= 0 && seq < h->max_seqs && layer >= 0 && layer < c.n_layers, "index out of range");
    TL_REQ(h, pos >= 0 && pos < c.max_pos, "position out of range");
    TL_REQ(h, x, "null pointer");
    if (!h->layers[layer].wqkv) return fail(h, TL_ERR_BAD_DESCRIPTOR, "layer not loaded");
    int32_t r = upload_rows(h, 1, seq, false, pos);
    if (r) return r;
    TL_HIP(h, hipMemcpyAsync(h->x, x, sizeof(float) * h->D, hipMemcpyDeviceToDevice, h->stream));
    if ((r = layer_rows(h, layer, 1, pos + 1, true))) return r;
    TL_HIP(h, hipMemcpyAsync(x, h->x, sizeof(float) * h->D, hipMemcpyDeviceToDevice, h->stream));
    return finish(h);
}

}  // extern "C"

namespace {

// embedding + all layers over n prompt tokens of sequence seq (positions
// 0..n-1); leaves the final hidden rows in h->x
// With abort_flag, the layers are launched one at a time: layer l + 1 goes out
// after layer l has finished and the flag has been read (prefill_decode_
// controller.sv takes HOST_ABORT in every state); *aborted reports a stop.
int32_t prefill_layers(tl_handle* h, int32_t seq, const int32_t* tokens, int32_t n,
                       const volatile int32_t* abort_flag = nullptr, bool* aborted = nullptr) {
    const tl_config& c = h->cfg;
    TL_REQ(h, seq >= 0 && seq < h->max_seqs, "sequence out of range");
    TL_REQ(h, tokens && n >= 1, "Input token sequence is empty");
    TL_REQ(h, n <= c.max_pos, "Sequence length exceeds max_position_embeddings");
    for (int i = 0; i < n; i++) TL_REQ(h, tokens[i] >= 0 && tokens[i] < c.vocab, "token id out of range");
    int32_t r = check_model_loaded(h);
    if (r) return r;
    h->host_ngen[seq] = 0;   // the sequence is rewritten: no decode until prefill_finish
    h->host_cursor[seq] = 0;
    if ((r = upload_rows(h, n, seq, false, 0))) return r;
    TL_HIP(h, hipMemcpyAsync(h->tokens, tokens, sizeof(int32_t) * n, hipMemcpyHostToDevice, h->stream));
    const int32_t zero = 0;
    TL_HIP(h, hipMemcpyAsync(h->n_gen + seq, &zero, sizeof zero, hipMemcpyHostToDevice, h->stream));
    TL_HIP(h, hipMemcpyAsync(h->cursor + seq, &n, sizeof n, hipMemcpyHostToDevice, h->stream));
    TL_LAUNCH(h, launch_reset_keys(h->stream, h->keys + seq, 1));
    if ((r = set_stop_state(h, seq, -1))) return r;
    TL_LAUNCH(h, launch_embed(h->stream, h->tokens, n, h->D, h->cfg.vocab, h->emb, h->emb_s, h->x));
    for (int l = 0; l < c.n_layers; l++) {
        if (abort_flag) {
            if (l > 0) {
                hipEvent_t ev = h->watch_ev[0];
                hipError_t q;
                while ((q = hipEventQuery(ev)) == hipErrorNotReady) {
                    if (*abort_flag) break;
                    std::this_thread::sleep_for(std::chrono::microseconds(10));
                }
                if (q != hipErrorNotReady) TL_HIP(h, q);
            }
            if (*abort_flag) {
                if (aborted) *aborted = true;
                return finish(h);
            }
        }
        if ((r = layer_rows(h, l, n, n, false))) return r;
        if (abort_flag) TL_HIP(h, hipEventRecord(h->watch_ev[0], h->stream));
    }
    return TL_OK;
}

// next-token bookkeeping from the last prompt row, then wait and report
int32_t prefill_finish(tl_handle* h, int32_t seq, int32_t n, int32_t* next_token, float* next_logit) {
    const tl_config& c = h->cfg;
    int32_t r;
    if ((r = lm_head_rows(h, h->x + (size_t)(n - 1) * h->D, 1, seq, 0))) return r;
    if ((r = finish(h))) return r;
    h->host_cursor[seq] = n;
    h->host_ngen[seq] = 1;
    if (next_token) TL_HIP(h, hipMemcpy(next_token, h->tokens_out + (size_t)seq * c.max_pos, sizeof(int32_t), hipMemcpyDeviceToHost));
    if (next_logit) TL_HIP(h, hipMemcpy(next_logit, h->logit_out + (size_t)seq * c.max_pos, sizeof(float), hipMemcpyDeviceToHost));
    return TL_OK;
}

}  // namespace

extern "C" {

int32_t tl_prefill(tl_handle* h, int32_t seq, const int32_t* tokens, int32_t n, int32_t* next_token, float* next_logit) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    int32_t r = prefill_layers(h, seq, tokens, n);
    if (r) return r;
    return prefill_finish(h, seq, n, next_token, next_logit);
}

int32_t tl_prefill_logits(tl_handle* h, int32_t seq, const int32_t* tokens, int32_t n, float* logits) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, logits, "null pointer");
    int32_t r = prefill_layers(h, seq, tokens, n);
    if (r) return r;
    const tl_config& c = h->cfg;
    {
        Prof p(h, TL_K_NORM, (double)n * h->D * 9.0);
        TL_LAUNCH(h, launch_rmsnorm_quant(h->stream, h->x, h->g_final, n, h->D, c.rms_eps, h->plan, nullptr, h->a8, h->as));
    }
    GemmArgs a{};
    a.a = h->a8; a.w = h->lm_w; a.as = h->as; a.ws = h->lm_s; a.y = logits; a.m = n; a.n = c.vocab; a.k = h->D;
    if ((r = run_gemm(h, EPI_DEQUANT, a, TL_K_LMHEAD))) return r;
    return prefill_finish(h, seq, n, nullptr, nullptr);
}

int32_t tl_layer_rows(tl_handle* h, int32_t seq, int32_t layer, int32_t pos0, int32_t rows, float* x) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    const tl_config& c = h->cfg;
    TL_REQ(h, seq >= 0 && seq < h->max_seqs && layer >= 0 && layer < c.n_layers, "index out of range");
    TL_REQ(h, rows >= 1 && rows <= h->max_rows, "row count out of range");
    TL_REQ(h, pos0 >= 0 && (int64_t)pos0 + rows <= c.max_pos, "Sequence length exceeds max_position_embeddings");
    TL_REQ(h, x, "null pointer");
    if (!h->layers[layer].wqkv) return fail(h, TL_ERR_BAD_DESCRIPTOR, "layer not loaded");
    int32_t r = upload_rows(h, rows, seq, false, pos0);
    if (r) return r;
    TL_HIP(h, hipMemcpyAsync(h->x, x, sizeof(float) * h->D * rows, hipMemcpyDeviceToDevice, h->stream));
    if ((r = layer_rows(h, layer, rows, pos0 + rows, rows == 1))) return r;
    TL_HIP(h, hipMemcpyAsync(x, h->x, sizeof(float) * h->D * rows, hipMemcpyDeviceToDevice, h->stream));
    return finish(h);
}

int32_t tl_dequantize_i32(tl_handle* h, const int32_t* acc, int64_t rows, int32_t cols, double input_scale,
                          double weight_scale, const float* bias, float* y) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, acc && y && rows >= 0 && cols > 0, "bad dequantize arguments");
    const float m = (float)(input_scale * weight_scale);
    TL_LAUNCH(h, launch_dequant_i32(h->stream, acc, rows * cols, cols, m, bias, y));
    return finish(h);
}

int32_t tl_decode(tl_handle* h, int32_t seq, int32_t max_new, int32_t eos_id, const volatile int32_t* abort_flag,
                  int32_t* tokens_out, int32_t* n_out, int32_t* stop_reason) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    const tl_config& c = h->cfg;
    TL_REQ(h, seq >= 0 && seq < h->max_seqs, "sequence out of range");
    TL_REQ(h, max_new >= 1, "--max-tokens must be at least 1");
    TL_REQ(h, tokens_out && n_out, "null pointer");
    TL_REQ(h, h->host_ngen[seq] >= 1, "tl_decode needs a prefilled sequence");
    TL_REQ(h, (int64_t)h->host_cursor[seq] + max_new <= c.max_pos, "Sequence length exceeds max_position_embeddings");
    *n_out = 0;
    if (stop_reason) *stop_reason = TL_STOP_NONE;
    const int32_t first = h->host_ngen[seq];
    int32_t r;
    if ((r = set_stop_state(h, seq, eos_id))) return r;
    if ((r = upload_rows(h, 1, seq, false, h->host_cursor[seq]))) return r;
    if ((r = decode_embed1(h))) return r;
    auto launch_step = [&](int32_t i) -> int32_t {
        if (!h->profiling) return decode_graph_launch(h, seq);
        return decode_step1(h, seq, h->host_cursor[seq] + i + 1);   // profiling: direct launches
    };
    volatile int32_t* abort_word = h->ctl_host;
    volatile int32_t* stop_mirror = h->ctl_host + 1 + seq;
    AbortWordReset reset_abort{h};
    *abort_word = 0;
    *stop_mirror = 0;
    const bool watch = eos_id >= 0 || abort_flag;
    int32_t launched = 0;
    bool abort_sent = false;
    if (!watch) {
        for (; launched < max_new; launched++)
            if ((r = launch_step(launched))) return r;
    } else {
        // kWatchDepth steps in flight: the host waits for the oldest, polling
        // the caller's abort flag, and after every step reads the mirror of the
        // device's stop flag.  A raised abort flag goes to the abort word the
        // token bookkeeping kernel reads, so the steps still in flight record
        // nothing from then on (at most the step whose bookkeeping already ran
        // records its token), and no further step is launched.
        auto poll_abort = [&]() {
            if (!abort_sent && abort_flag && *abort_flag) {
                *abort_word = 1;
                abort_sent = true;
            }
        };
        poll_abort();
        int32_t done = 0, dev_stop = 0;
        for (;;) {
            while (!abort_sent && dev_stop == 0 && launched < max_new && launched - done < kWatchDepth) {
                if ((r = launch_step(launched))) return r;
                TL_HIP(h, hipEventRecord(h->watch_ev[launched % kWatchDepth], h->stream));
                launched++;
            }
            if (done == launched) break;
            hipError_t q;
            while ((q = hipEventQuery(h->watch_ev[done % kWatchDepth])) == hipErrorNotReady) {
                poll_abort();
                std::this_thread::sleep_for(std::chrono::microseconds(20));
            }
            TL_HIP(h, q);
            done++;
            dev_stop = *stop_mirror;
            poll_abort();
        }
    }
    int32_t ngen = 0;
    TL_HIP(h, hipMemcpyAsync(&ngen, h->n_gen + seq, sizeof ngen, hipMemcpyDeviceToHost, h->stream));
    if ((r = finish(h))) return r;
    const int32_t got = ngen - first;
    if (got < 0 || got > launched) return fail(h, TL_ERR_INTERNAL, "decode: device token count out of range");
    h->host_cursor[seq] += got;
    h->host_ngen[seq] += got;
    *n_out = got;
    if (got > 0)
        TL_HIP(h, hipMemcpy(tokens_out, h->tokens_out + (size_t)seq * c.max_pos + first, sizeof(int32_t) * got,
                            hipMemcpyDeviceToHost));
    // 1: the device recorded EOS (and then stopped checking); 2: it saw the
    // abort word first; an abort raised before any step ran records nothing
    const int32_t dstop = watch ? *stop_mirror : 0;
    if (stop_reason)
        *stop_reason = dstop == 1   ? TL_STOP_EOS
                       : dstop == 2 ? TL_STOP_HOST_ABORT
                                    : (abort_sent && got < max_new ? TL_STOP_HOST_ABORT : TL_STOP_MAX_TOKENS);
    return TL_OK;
}

int32_t tl_generate(tl_handle* h, int32_t seq, const int32_t* prompt, int32_t n_prompt, int32_t max_new, int32_t eos_id,
                    const volatile int32_t* abort_flag, int32_t* tokens_out, int32_t* n_out, int32_t* stop_reason) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    TL_REQ(h, max_new >= 1, "--max-tokens must be at least 1");
    TL_REQ(h, tokens_out && n_out, "null pointer");
    TL_REQ(h, prompt && n_prompt >= 1, "Input token sequence is empty");
    TL_REQ(h, (int64_t)n_prompt + max_new - 1 <= h->cfg.max_pos, "Sequence length exceeds max_position_embeddings");
    *n_out = 0;
    if (stop_reason) *stop_reason = TL_STOP_NONE;
    if (abort_flag && *abort_flag) {
        if (stop_reason) *stop_reason = TL_STOP_HOST_ABORT;
        return TL_OK;
    }
    int32_t first = 0;
    bool aborted = false;
    int32_t r = prefill_layers(h, seq, prompt, n_prompt, abort_flag, &aborted);
    if (r) return r;
    if (aborted) {
        if (stop_reason) *stop_reason = TL_STOP_HOST_ABORT;
        return TL_OK;
    }
    if ((r = prefill_finish(h, seq, n_prompt, &first, nullptr))) return r;
    tokens_out[0] = first;
    *n_out = 1;
    if (eos_id >= 0 && first == eos_id) {
        if (stop_reason) *stop_reason = TL_STOP_EOS;
        return TL_OK;
    }
    if (max_new == 1) {
        if (stop_reason) *stop_reason = TL_STOP_MAX_TOKENS;
        return TL_OK;
    }
    int32_t more = 0;
    r = tl_decode(h, seq, max_new - 1, eos_id, abort_flag, tokens_out + 1, &more, stop_reason);
    *n_out = 1 + more;
    return r;
}

int32_t tl_decode_batch(tl_handle* h, int32_t n_seqs, const int32_t* tokens, const int32_t* start_pos, int32_t n_steps,
                        int32_t* tokens_out) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    const tl_config& c = h->cfg;
    TL_REQ(h, n_seqs >= 1 && n_seqs <= h->max_seqs, "batch larger than max_seqs");
    TL_REQ(h, tokens && start_pos && tokens_out && n_steps >= 1, "bad decode_batch arguments");
    int32_t max_t = 0;
    for (int b = 0; b < n_seqs; b++) {
        TL_REQ(h, tokens[b] >= 0 && tokens[b] < c.vocab, "token id out of range");
        TL_REQ(h, start_pos[b] >= 0 && (int64_t)start_pos[b] + n_steps <= c.max_pos,
               "Sequence length exceeds max_position_embeddings");
        max_t = std::max(max_t, start_pos[b] + n_steps);
    }
    int32_t r = check_model_loaded(h);
    if (r) return r;
    if ((r = upload_rows(h, n_seqs, 0, true, 0))) return r;
    std::vector<int32_t> zeros(n_seqs, 0);
    TL_HIP(h, hipMemcpyAsync(h->token_cur, tokens, sizeof(int32_t) * n_seqs, hipMemcpyHostToDevice, h->stream));
    TL_HIP(h, hipMemcpyAsync(h->cursor, start_pos, sizeof(int32_t) * n_seqs, hipMemcpyHostToDevice, h->stream));
    TL_HIP(h, hipMemcpyAsync(h->n_gen, zeros.data(), sizeof(int32_t) * n_seqs, hipMemcpyHostToDevice, h->stream));
    TL_LAUNCH(h, launch_reset_keys(h->stream, h->keys, n_seqs));
    // the first step runs eagerly (it sizes the scratch the LM head's tile
    // keys need), the rest replay the captured step
    for (int step = 0; step < n_steps; step++) {
        if (step > 0 && !h->profiling) {
            if ((r = batch_graph_launch(h, n_seqs))) return r;
        } else if ((r = batch_step(h, n_seqs, max_t))) {
            return r;
        }
    }
    if ((r = finish(h))) return r;
    for (int b = 0; b < n_seqs; b++) {
        TL_HIP(h, hipMemcpy(tokens_out + (size_t)b * n_steps, h->tokens_out + (size_t)b * c.max_pos,
                            sizeof(int32_t) * n_steps, hipMemcpyDeviceToHost));
        h->host_cursor[b] = start_pos[b] + n_steps;
        h->host_ngen[b] = n_steps;
    }
    return TL_OK;
}

// ---- debug capture -------------------------------------------------------------------

}  // extern "C"

namespace {

// device buffers of one capture, freed after the stream has drained
struct CaptureScratch {
    hipStream_t stream;
    std::vector<void*> ptrs;
    explicit CaptureScratch(hipStream_t s) : stream(s) {}
    ~CaptureScratch() {
        (void)hipStreamSynchronize(stream);
        for (void* p : ptrs) (void)hipFree(p);
    }
    template <class T>
    T* get(size_t n) {
        void* p = nullptr;
        if (hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)) != hipSuccess) return nullptr;
        ptrs.push_back(p);
        return (T*)p;
    }
};

// device -> host copy on the handle's stream when the destination is wanted
hipError_t copy_out(tl_handle* h, void* dst, const void* src, size_t bytes) {
    if (!dst || !bytes) return hipSuccess;
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, h->stream);
}

// the capture layer's tensors once its decode kernels have run: the layer's
// input was saved in xin; the attention input and the query are quantized
// again, and the window's scores and probabilities are recomputed, by the
// per-row kernels of the prefill path from the layer's Q|K|V (h->qkv)
int32_t capture_layer(tl_handle* h, int32_t layer, int32_t pos, const float* xin, tl_capture* cap, CaptureScratch& sc) {
    const tl_config& c = h->cfg;
    const int D = h->D, KVD = h->KVD, Hq = c.n_heads, Hkv = c.n_kv_heads;
    const LayerDev& L = h->layers[layer];
    int8_t* a8 = sc.get<int8_t>(D);
    double* as = sc.get<double>(1);
    int8_t* kv_rows = sc.get<int8_t>(2 * (size_t)KVD);
    const size_t win = (size_t)Hq * cap->n_keys;
    int32_t* scores = sc.get<int32_t>(win);
    int8_t* probs = sc.get<int8_t>(win);
    float* scl = sc.get<float>(Hq);
    if (!a8 || !as || !kv_rows || !scores || !probs || !scl) return fail(h, TL_ERR_INTERNAL, "hipMalloc");
    TL_HIP(h, copy_out(h, cap->qkv, h->qkv, sizeof(float) * h->QKV));
    TL_HIP(h, copy_out(h, cap->attended, h->att, sizeof(float) * D));
    TL_HIP(h, copy_out(h, cap->layer_out, h->x, sizeof(float) * D));
    TL_LAUNCH(h, launch_rmsnorm_quant(h->stream, xin, L.g_in, 1, D, c.rms_eps, h->plan, nullptr, a8, as));
    TL_HIP(h, copy_out(h, cap->attn_in_q, a8, D));
    TL_HIP(h, copy_out(h, &cap->attn_in_scale, as, sizeof(double)));
    for (int g = 0; g < Hkv; g++)
        TL_LAUNCH(h, launch_kv_gather(h->stream, h->kv, h->rows_seq, layer, g, pos, 1, kv_rows + g * kHeadDim,
                                      kv_rows + KVD + g * kHeadDim));
    TL_HIP(h, copy_out(h, cap->k_row, kv_rows, KVD));
    TL_HIP(h, copy_out(h, cap->v_row, kv_rows + KVD, KVD));
    if (cap->kv_scales) {
        TL_HIP(h, copy_out(h, cap->kv_scales, h->kv_sk + (size_t)layer * Hkv, sizeof(float) * Hkv));
        TL_HIP(h, copy_out(h, cap->kv_scales + Hkv, h->kv_sv + (size_t)layer * Hkv, sizeof(float) * Hkv));
    }
    TL_LAUNCH(h, launch_qkv_post(h->stream, h->qkv, 1, Hq, Hkv, rowmap(h), h->rope_cos, h->rope_sin, h->kv, layer,
                                 h->kv_sk, h->kv_sv, h->q8, h->qs, nullptr, false));
    TL_HIP(h, copy_out(h, cap->q8, h->q8, D));
    TL_HIP(h, copy_out(h, &cap->q_scale, h->qs, sizeof(double)));
    AttnDebug dbg;
    dbg.scores = scores;
    dbg.probs = probs;
    dbg.score_scale = scl;
    dbg.key0 = cap->key0;
    dbg.n_keys = cap->n_keys;
    // the recomputed attention output goes to h->att, whose copy is queued above
    TL_LAUNCH(h, launch_attention(h->stream, h->q8, h->qs, 1, Hq, Hkv, rowmap(h), h->kv, layer, h->kv_sk, h->kv_sv,
                                  h->att, pos + 1, dbg));
    TL_HIP(h, copy_out(h, cap->score_scale, scl, sizeof(float) * Hq));
    TL_HIP(h, copy_out(h, cap->scores, scores, sizeof(int32_t) * win));
    TL_HIP(h, copy_out(h, cap->probs, probs, win));
    return TL_OK;
}

}  // namespace

extern "C" {

int32_t tl_capture_step(tl_handle* h, int32_t seq, tl_capture* cap) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    const tl_config& c = h->cfg;
    TL_REQ(h, cap, "null pointer");
    TL_REQ(h, seq >= 0 && seq < h->max_seqs, "sequence out of range");
    TL_REQ(h, cap->layer >= 0 && cap->layer < c.n_layers, "capture layer out of range");
    TL_REQ(h, h->host_ngen[seq] >= 1, "tl_capture_step needs a prefilled sequence");
    const int32_t pos = h->host_cursor[seq];
    TL_REQ(h, pos + 1 <= c.max_pos, "Sequence length exceeds max_position_embeddings");
    TL_REQ(h, cap->key0 >= 0 && cap->key0 <= pos + 1, "attention window outside keys 0..pos");
    if (cap->n_keys < 0) cap->n_keys = pos + 1 - cap->key0;
    TL_REQ(h, cap->n_keys >= 0 && (int64_t)cap->key0 + cap->n_keys <= pos + 1, "attention window outside keys 0..pos");
    int32_t r = check_model_loaded(h);
    if (r) return r;
    if ((r = set_stop_state(h, seq, -1))) return r;
    const int D = h->D, V = c.vocab;
    const int32_t first = h->host_ngen[seq];
    CaptureScratch sc(h->stream);
    float* xin = sc.get<float>(D);
    if (!xin) return fail(h, TL_ERR_INTERNAL, "hipMalloc");
    if ((r = upload_rows(h, 1, seq, false, pos))) return r;
    cap->pos = pos;
    TL_HIP(h, hipMemcpyAsync(&cap->token_in, h->token_cur + seq, sizeof(int32_t), hipMemcpyDeviceToHost, h->stream));
    // one step of decode_step1, eagerly
    TL_LAUNCH(h, launch_embed_step(h->stream, h->token_cur, h->row_seq, 1, h->cursor, h->row_pos, h->D, c.vocab,
                                   h->emb, h->emb_s, h->x));
    for (int l = 0; l < c.n_layers; l++) {
        if (l == cap->layer) {
            TL_HIP(h, hipMemcpyAsync(xin, h->x, sizeof(float) * D, hipMemcpyDeviceToDevice, h->stream));
            TL_HIP(h, copy_out(h, cap->layer_in, h->x, sizeof(float) * D));
        }
        if ((r = layer_row1(h, l, pos + 1))) return r;
        if (l == cap->layer && (r = capture_layer(h, l, pos, xin, cap, sc))) return r;
    }
    TL_HIP(h, copy_out(h, cap->final_hidden, h->x, sizeof(float) * D));
    std::vector<float> logits;
    if (cap->top_ids || cap->top_logits) {
        // the step's logits through the standalone LM-head operator's kernels
        logits.resize(V);
        TL_LAUNCH(h, launch_reset_keys(h->stream, h->op_key, 1));
        TL_LAUNCH(h, launch_rmsnorm_quant(h->stream, h->x, h->g_final, 1, D, c.rms_eps, h->plan, nullptr, h->a8, h->as));
        GemvArgs g{};
        g.w = h->lm_w; g.ws = h->lm_s; g.x = h->a8; g.xs = h->as; g.key = h->op_key; g.y = h->logits; g.n = V; g.k = D;
        TL_LAUNCH(h, launch_gemv(h->stream, EPI_ARGMAX, g));
        TL_HIP(h, copy_out(h, logits.data(), h->logits, sizeof(float) * V));
    }
    if ((r = lm_head_rows(h, h->x, 1, seq, 1))) return r;
    const size_t slot = (size_t)seq * c.max_pos + first;
    TL_HIP(h, hipMemcpyAsync(&cap->token, h->tokens_out + slot, sizeof(int32_t), hipMemcpyDeviceToHost, h->stream));
    TL_HIP(h, hipMemcpyAsync(&cap->logit, h->logit_out + slot, sizeof(float), hipMemcpyDeviceToHost, h->stream));
    if ((r = finish(h))) return r;
    h->host_cursor[seq] += 1;
    h->host_ngen[seq] += 1;
    if (!logits.empty()) {
        const int k = std::min(TL_CAPTURE_TOPK, V);
        std::vector<int32_t> idx(V);
        for (int i = 0; i < V; i++) idx[i] = i;
        std::partial_sort(idx.begin(), idx.begin() + k, idx.end(), [&](int32_t a, int32_t b) {
            return logits[a] > logits[b] || (logits[a] == logits[b] && a < b);
        });
        for (int i = 0; i < k; i++) {
            if (cap->top_ids) cap->top_ids[i] = idx[i];
            if (cap->top_logits) cap->top_logits[i] = logits[idx[i]];
        }
    }
    return TL_OK;
}

// ---- profiling -----------------------------------------------------------------------

int32_t tl_set_profiling(tl_handle* h, int32_t on) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    harvest_profile(h);
    h->profiling = on != 0;
    for (int i = 0; i < TL_K_COUNT; i++) {
        h->prof_count[i] = 0;
        h->prof_ms[i] = 0.0;
        h->prof_bytes[i] = 0.0;
    }
    return TL_OK;
}

int32_t tl_get_profile(tl_handle* h, int32_t kclass, int64_t* count, double* total_ms, double* bytes) {
    if (!h || kclass < 0 || kclass >= TL_K_COUNT) return TL_ERR_BAD_DESCRIPTOR;
    harvest_profile(h);
    if (count) *count = h->prof_count[kclass];
    if (total_ms) *total_ms = h->prof_ms[kclass];
    if (bytes) *bytes = h->prof_bytes[kclass];
    return TL_OK;
}

int32_t tl_decode_timeline(tl_handle* h, int32_t seq, int32_t n_steps, tl_timeline* out) {
    if (!h) return TL_ERR_BAD_DESCRIPTOR;
    const tl_config& c = h->cfg;
    TL_REQ(h, out && n_steps >= 1, "bad timeline arguments");
    TL_REQ(h, seq >= 0 && seq < h->max_seqs, "sequence out of range");
    TL_REQ(h, h->host_ngen[seq] >= 1, "tl_decode_timeline needs a prefilled sequence");
    TL_REQ(h, (int64_t)h->host_cursor[seq] + n_steps <= c.max_pos, "Sequence length exceeds max_position_embeddings");
    int32_t r = check_model_loaded(h);
    if (r) return r;
    int rate_khz = 0;
    TL_HIP(h, hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, h->device));
    TL_REQ(h, rate_khz > 0, "device reports no wall-clock rate");
    if (!h->ts_buf) {
        h->ts_cap = (size_t)1 << 22;
        TL_HIP(h, dalloc(h, &h->ts_buf, h->ts_cap));
    }
    if ((r = set_stop_state(h, seq, -1))) return r;
    if ((r = upload_rows(h, 1, seq, false, h->host_cursor[seq]))) return r;
    if ((r = decode_embed1(h))) return r;
    // capture one step with stamp regions
    h->ts_on = true;
    h->ts_overflow = false;
    h->ts_used = 0;
    h->ts_slots.clear();
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamBeginCapture(h->stream, hipStreamCaptureModeThreadLocal);
    if (e == hipSuccess) {
        r = decode_step1(h, seq, c.max_pos);
        e = hipStreamEndCapture(h->stream, &graph);
    }
    h->ts_on = false;
    if (r || e != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        return r ? r : fail(h, TL_ERR_INTERNAL, std::string("timeline capture: ") + hipGetErrorString(e));
    }
    if (h->ts_overflow) {
        (void)hipGraphDestroy(graph);
        return fail(h, TL_ERR_INTERNAL, "timeline stamp buffer too small");
    }
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    TL_HIP(h, e);
    std::vector<unsigned long long> st(h->ts_used);
    *out = tl_timeline{};
    const double us_per_tick = 1000.0 / (double)rate_khz;
    int32_t done = 0;
    for (; done < n_steps; done++) {
        e = hipMemsetAsync(h->ts_buf, 0, h->ts_used * sizeof(unsigned long long), h->stream);
        if (e == hipSuccess) e = hipGraphLaunch(exec, h->stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(st.data(), h->ts_buf, h->ts_used * sizeof(unsigned long long), hipMemcpyDeviceToHost,
                               h->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(h->stream);
        if (e != hipSuccess) break;
        // per kernel: first wavefront start, last wavefront end (unstamped
        // wavefronts, e.g. past the end of a grid, hold zeros)
        unsigned long long first = 0, last = 0, prev_end = 0;
        int prev_class = -1, kernels = 0;
        for (const auto& sl : h->ts_slots) {
            unsigned long long a = ~0ull, b = 0;
            for (int64_t w = 0; w < sl.waves; w++) {
                const unsigned long long t0 = st[sl.off + 2 * w], t1 = st[sl.off + 2 * w + 1];
                if (t1 == 0) continue;
                a = std::min(a, t0);
                b = std::max(b, t1);
            }
            if (b == 0) continue;
            kernels++;
            out->busy_us[sl.kclass] += (double)(b - a) * us_per_tick;
            out->launches[sl.kclass] += 1;
            if (prev_class >= 0) out->gap_us[prev_class] += ((double)a - (double)prev_end) * us_per_tick;
            if (!first) first = a;
            last = b;
            prev_end = b;
            prev_class = sl.kclass;
        }
        out->kernels = kernels;
        out->step_us += (double)(last - first) * us_per_tick;
    }
    (void)hipGraphExecDestroy(exec);
    // the steps that ran are ordinary decode steps
    h->host_cursor[seq] += done;
    h->host_ngen[seq] += done;
    TL_HIP(h, e);
    out->steps = done;
    const double inv = 1.0 / (double)std::max(done, 1);
    out->step_us *= inv;
    for (int k = 0; k < TL_K_COUNT; k++) {
        out->busy_us[k] *= inv;
        out->gap_us[k] *= inv;
        out->launches[k] = (int32_t)((out->launches[k] + done / 2) / std::max(done, 1));
    }
    return TL_OK;
}

}  // extern "C"
