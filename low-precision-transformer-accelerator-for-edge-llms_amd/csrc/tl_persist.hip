// tl_persist.hip -- batch-1 greedy decode steps as ONE persistent kernel.
//
// The per-layer kernels of tl_decode.hip pay a fixed ~3-4 us per launch (wave
// ramp, first bytes from HBM, prologue, epilogue) on top of the weight
// stream; at 5 launches x 22 layers that fixed part is most of a decode step.
// Here one cooperative launch (one 256-thread workgroup per CU, all
// co-resident) runs every phase of every layer of several steps:
//
//   P1  x -> RMSNorm -> INT8 -> Q|K|V rows           (all workgroups)
//   P2  RoPE, Q/K/V quantization, KV append, INT8 GQA attention
//                                                     (one workgroup per query head)
//   P3  attended -> INT8 -> O rows + residual         (all)
//   P4  x -> RMSNorm -> INT8 -> gate/up rows, SiLU(gate) * up   (all)
//   P5  hidden -> INT8 -> down rows + residual        (all)
//   P6  final RMSNorm -> LM head rows -> argmax key   (all), then every
//       workgroup reads the step's token
//
// There are no grid barriers.  A phase's outputs are stored with agent-scope
// (write-through) stores; each producing workgroup then waits for its stores
// to complete and adds one to the phase's counter (sliced by XCD: 8 counters
// on separate cache lines, so each takes ~1/8 of the atomics).  Wavefront 0
// of each workgroup is its control wavefront and holds no weight rows: it
// polls the 8 slices until they add up to the number of producers the phase
// has had so far, then copies the whole input vector into LDS with
// agent-scope loads: one round trip, and a few hundred polls per phase rather
// than one per element.  Wavefronts 1..3 issue the weight loads of their rows
// before the wait (O with gate/up, down with the next layer's Q|K|V), so the
// weight stream overlaps the dependency, and the memory counter of the
// polling wavefront never waits behind it.
// Buffers are reused every layer; every reuse is ordered after all reads of
// the previous contents because each RMSNorm (and the O and down
// projections) consumes a whole vector, i.e. depends on every producer of
// the phase before.  KV rows are
// written with agent-scope (write-through) stores and read with agent-scope
// loads, so rows written in earlier steps are never read from a stale cache.
// Every wait is bounded: past the limit the workgroup sets an error flag and
// leaves, and every other workgroup leaves at its next wait.
//
// The arithmetic is that of the per-layer kernels (same prologues, same
// reduction orders, same epilogues), so tokens, logits and KV rows are
// bit-identical to them and to the CPU oracle.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "tl_device.h"
#include "tl_internal.h"
#include "tl_prologue.h"

namespace tl {

namespace {

constexpr unsigned kSpinLimit = 1u << 20;   // polls (each >= one memory round trip) before giving up

TL_DEV void putf(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
TL_DEV float getf(const float* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
TL_DEV unsigned peek32(const unsigned* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// four consecutive floats through the coherence point (two 64-bit loads)
TL_DEV float4 getf4(const float* p) {
    const uint64_t a = __hip_atomic_load((const uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t b = __hip_atomic_load((const uint64_t*)p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float4(__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)),
                       __uint_as_float((uint32_t)b), __uint_as_float((uint32_t)(b >> 32)));
}

// 16 bytes of the KV cache through the coherence point (two 64-bit loads)
TL_DEV v4i ldc16(const int8_t* p) {
    const uint64_t a = __hip_atomic_load((const uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t b = __hip_atomic_load((const uint64_t*)p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    v4i r;
    r[0] = (int)(uint32_t)a;
    r[1] = (int)(uint32_t)(a >> 32);
    r[2] = (int)(uint32_t)b;
    r[3] = (int)(uint32_t)(b >> 32);
    return r;
}

typedef __attribute__((address_space(1))) void GlobalVoid;
typedef __attribute__((address_space(3))) void LdsVoid;
constexpr int kCoherentLoad = 16;   // cache policy of a device-scope coherent load (sc1)

constexpr int kSlices = 8;          // counter slices (one per XCD)
constexpr int kSliceStride = 32;    // unsigned words: one 128-byte line per slice

// this workgroup's outputs of `phase` are complete: count it in
TL_DEV void signal_phase(unsigned* ctr, int phase) {
    __builtin_amdgcn_s_waitcnt(0);   // this thread's stores have reached the coherence point
    __syncthreads();                 // ... and every other thread's
    if (threadIdx.x == 0)
        __hip_atomic_fetch_add(ctr + (phase * kSlices + (blockIdx.x & (kSlices - 1))) * kSliceStride, 1u,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

namespace {

// The launch's arguments and layer table are read-only while it runs: read
// them through the constant address space, so they come in with scalar loads
// (no wait behind the vector memory counter).  The kernel hands its kernarg
// segment pointer to the phase functions (the builtin itself is defined in
// kernels only); a callee's arguments arrive in vector registers, so it makes
// the pointer wave-uniform again before use.
typedef __attribute__((address_space(4))) const PersistArgs KArgs;
typedef __attribute__((address_space(4))) const PLayer KLayer;
TL_DEV KArgs& uniform_args(KArgs* p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return *(KArgs*)(((uint64_t)hi << 32) | lo);
}
TL_DEV KLayer& klayer(KArgs& a, int l) { return ((KLayer*)a.layers)[l]; }

constexpr int kPhases = 8;
constexpr int kQkvPerThread = 12;   // Q|K|V width <= 12 x 256 floats
enum { PH_QKV = 0, PH_ATT = 1, PH_O = 2, PH_GLU = 3, PH_DOWN = 4 };
// producer count of `phase` once it has run for (step, layer) and everything before
TL_DEV unsigned ptarget(KArgs& a, int step, int layer, int phase) {
    const unsigned runs = (unsigned)(step * a.n_layers + layer + 1);
    return runs * (phase == PH_ATT ? (unsigned)a.H : (unsigned)gridDim.x);
}

// LDS of one workgroup; phases use it one after another
struct Lds {
    int8_t* xs8;      // [6 KiB]   INT8 activation row
    float* sq;        // [2048]    squares for RMSNorm
    float* part;      // [512]
    float* red;       // [16]
    double* xscale;   // [1]
    unsigned long long* wbest;  // [4]
    float* att;       // attention scratch (rest of the buffer)
};

// the embedding row of token tok (f32(e8) * s_e), same chunking
template <int KCH>
TL_DEV void load_embedding(KArgs& a, int tok, float4 (&xv)[KCH]) {
    const int tid = threadIdx.x;
    const float s = a.emb_s[tok];
    const int8_t* e8 = a.emb + (int64_t)tok * a.D;
#pragma unroll
    for (int c = 0; c < KCH; c++) {
        const int e = (c * kNT + tid) * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (e < a.D) {
            v.x = (float)e8[e] * s;
            v.y = (float)e8[e + 1] * s;
            v.z = (float)e8[e + 2] * s;
            v.w = (float)e8[e + 3] * s;
        }
        xv[c] = v;
    }
}

// one GEMV phase: every wavefront of the grid owns RB consecutive rows per
// round (rounds stride over the grid).  The first round's weights are loaded
// before the activation is awaited.  Epilogues as in the fused kernels.
struct GemvPhase {
    const int8_t* w;
    const int8_t* w2;
    const float* ws;
    const float* ws2;
    int n, k;
};

template <int NM, int RB, int KCH>
TL_DEV void load_rows(const GemvPhase& g, int r0, v4i (&wv)[NM][RB][KCH]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int m = 0; m < NM; m++) {
        const int8_t* wb = m ? g.w2 : g.w;
#pragma unroll
        for (int r = 0; r < RB; r++) {
            const int8_t* wr = wb + (int64_t)min(r0 + r, g.n - 1) * g.k;
#pragma unroll
            for (int c = 0; c < KCH; c++) wv[m][r][c] = ld_nt16(wr + min(c * 1024 + lane * 16, g.k - 16));
        }
    }
}

template <int NM, int RB, int KCH>
TL_DEV void dot_rows(const v4i (&wv)[NM][RB][KCH], const int8_t* xs8, int K, int (&mine)[NM]) {
    const int lane = threadIdx.x & 63;
    v4i xr[KCH];
#pragma unroll
    for (int c = 0; c < KCH; c++) {
        xr[c] = ld16(xs8 + c * 1024 + lane * 16);
        if (c * 1024 + lane * 16 >= K) xr[c] = (v4i){0, 0, 0, 0};
    }
#pragma unroll
    for (int m = 0; m < NM; m++) {
        int acc[RB];
#pragma unroll
        for (int r = 0; r < RB; r++) {
            int s = 0;
#pragma unroll
            for (int c = 0; c < KCH; c++) s = sdot4v(wv[m][r][c], xr[c], s);
            acc[r] = wave_sum_i32(s);
        }
        mine[m] = acc[0];
#pragma unroll
        for (int r = 1; r < RB; r++) mine[m] = lane == r ? acc[r] : mine[m];
    }
}

}  // namespace

TL_DEV Lds lds_map() {
    extern __shared__ __align__(16) unsigned char smem[];
    Lds L;
    L.xs8 = (int8_t*)smem;                                // 6 KiB
    L.sq = (float*)(smem + 6144);                         // 8 KiB
    L.part = (float*)(smem + 6144 + 8192);                // 2 KiB
    L.red = (float*)(smem + 6144 + 8192 + 2048);          // 64 B
    L.xscale = (double*)(smem + 6144 + 8192 + 2048 + 64); // 8 B
    L.wbest = (unsigned long long*)(smem + 6144 + 8192 + 2048 + 128);
    L.att = (float*)(smem + 6144 + 8192 + 2048 + 256);    // staged vector / attention scratch
    return L;
}

// Wavefront 0 is the control wavefront: it holds no weight rows, so its
// memory counter never waits behind the weight stream.  It polls the phase
// counters and copies each input vector into LDS with one round of
// agent-scope loads; wavefronts 1..3 own the weight rows.
// NIT: the most slices of 256 floats a K of this call site needs.  The copy
// goes straight from memory to LDS (16 bytes per lane, coherent at device
// scope), all slices in flight at once: one round trip, no registers.  LDS
// past K up to the slice end receives duplicates of the last elements.
template <int NIT>
TL_DEV bool wait_stage(KArgs& a, int phase, unsigned target, const float* src, int K, float* stage) {
    __shared__ int give_up;
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const unsigned* c = a.ctr + (phase * kSlices + (lane & (kSlices - 1))) * kSliceStride;
        bool ok = true;
        for (unsigned it = 0;; it++) {
            unsigned v = lane < kSlices ? peek32(c) : 0u;
#pragma unroll
            for (int off = 1; off < kSlices; off <<= 1) v += __shfl_xor(v, off);
            v = __shfl(v, 0);   // lanes 0..7 hold the total: every lane decides alike
            if (v >= target) break;
            if ((it & 63) == 63 && peek32(a.err)) { ok = false; break; }
            if (it >= kSpinLimit) {
                if (lane == 0) __hip_atomic_fetch_or(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (ok) {
#pragma unroll
            for (int i = 0; i < NIT; i++)
                if (i * 256 < K)
                    __builtin_amdgcn_global_load_lds((GlobalVoid*)(src + min(i * 256 + lane * 4, K - 4)),
                                                     (LdsVoid*)(stage + i * 256), 16, 0, kCoherentLoad);
            __builtin_amdgcn_s_waitcnt(0);
        }
        if (lane == 0) give_up = ok ? 0 : 1;
    }
    __syncthreads();
    return give_up == 0;
}

template <int KCH>
TL_DEV void chunks_from(const float* stage, int K, float4 (&xv)[KCH]) {
#pragma unroll
    for (int c = 0; c < KCH; c++) {
        const int e = (c * kNT + threadIdx.x) * 4;
        xv[c] = e < K ? *(const float4*)(stage + e) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

template <int KCH>
TL_DEV void gamma_chunks(const float* g, int K, float4 (&gv)[KCH]) {
#pragma unroll
    for (int c = 0; c < KCH; c++) {
        const int e = (c * kNT + threadIdx.x) * 4;
        gv[c] = e < K ? *(const float4*)(g + e) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

// first row of this wavefront's rows (waves 1..3), stride between rounds
TL_DEV int first_row(int rb) {
    const int wave = threadIdx.x >> 6;
    return wave ? (blockIdx.x * (kNW - 1) + wave - 1) * rb : 0x7fffffff;
}
TL_DEV int row_stride(int rb) { return gridDim.x * (kNW - 1) * rb; }

// One function per phase (not inlined: each gets its own register
// allocation).  false: a wait gave up, the caller leaves.

// P1 of layer 0: embedding -> RMSNorm -> Q|K|V rows
template <int KD>
__device__ __noinline__ bool ph_qkv0(KArgs* ap, int s, int tok) {
    KArgs& a = uniform_args(ap);
    s = __builtin_amdgcn_readfirstlane(s);
    tok = __builtin_amdgcn_readfirstlane(tok);
    const Lds L = lds_map();
    const int lane = threadIdx.x & 63;
    const int D = a.D, QKV = D + 2 * a.Hkv * kHeadDim;
    KLayer& Ly = klayer(a, 0);
    constexpr int RB = 4;
    GemvPhase g{Ly.wqkv, nullptr, Ly.sqkv, nullptr, QKV, D};
    v4i wv[1][RB][KD];
    int r0 = first_row(RB);
    if (r0 < QKV) load_rows<1, RB, KD>(g, r0, wv);
    float4 xv[KD], gv[KD];
    load_embedding<KD>(a, tok, xv);
    gamma_chunks<KD>(Ly.g_in, D, gv);
    prologue_rmsnorm<KD>(xv, gv, D, a.eps, PwPlan{a.plan.leaf_len, a.plan.n_leaves}, L.sq, L.part, L.xs8, L.red, L.xscale);
    const double sx = *L.xscale;
    for (; r0 < QKV; r0 += row_stride(RB)) {
        if (r0 != first_row(RB)) load_rows<1, RB, KD>(g, r0, wv);
        int mine[1];
        dot_rows<1, RB, KD>(wv, L.xs8, D, mine);
        const int n = r0 + lane;
        if (lane < RB && n < QKV) putf(a.t_qkv + n, (float)mine[0] * deq_mult(sx, g.ws[n]));
    }
    signal_phase(a.ctr, PH_QKV);
    (void)s;
    return true;
}

__device__ __noinline__ bool ph_att(KArgs* ap, int s, int layer, int pos) {
    KArgs& a = uniform_args(ap);
    s = __builtin_amdgcn_readfirstlane(s);
    layer = __builtin_amdgcn_readfirstlane(layer);
    pos = __builtin_amdgcn_readfirstlane(pos);
    const Lds L = lds_map();
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nwaves = gridDim.x * kNW, gw = blockIdx.x * kNW + wave;
    const int D = a.D, F = a.F, H = a.H, Hkv = a.Hkv, KVD = Hkv * kHeadDim, QKV = D + 2 * KVD;
    const int G = H / Hkv;
    unsigned* err = a.err;
    (void)lane; (void)nwaves; (void)gw; (void)F; (void)G; (void)QKV; (void)KVD;
    KLayer& Ly = klayer(a, layer);
    (void)Ly;
    // ---- P2: attention, one workgroup per query head ------------------
    {
        const int h = blockIdx.x, gk = h / G;
        const int T = pos + 1;
        const int tpad = (T + 63) & ~63, nblk = tpad >> 6, ngrp = tpad >> 4;
        float* v = L.att;                       // [QKV]
        float* s_buf = v + QKV;                 // [tpad]
        int8_t* p8 = (int8_t*)(s_buf + tpad);   // [tpad]
        float* bsum = (float*)(p8 + tpad);      // [nblk, padded to 4: qs stays 16-byte aligned]
        int8_t* qs = (int8_t*)(bsum + ((nblk + 3) & ~3));  // [64]
        int8_t* knew = qs + 64;                 // [64]
        int8_t* vnew = knew + 64;               // [64]
        float* misc = (float*)(vnew + 64);      // [16]: 0 scl, 1 mrow, 2 tot, 4.. wave max
        int* accs = (int*)(misc + 16);          // [4][64]
        const int64_t pl = KvGeom{nullptr, nullptr, a.kv.n_layers, a.kv.n_kv_heads, a.kv.max_pos}.plane(a.seq, layer, gk);
        const int8_t* kp = a.kv.k + pl;
        const int8_t* vp = a.kv.v + pl;
        const float cs = a.cosb[(int64_t)pos * kHeadDim + lane];
        const float sn = a.sinb[(int64_t)pos * kHeadDim + lane];
        if (!wait_stage<kQkvPerThread>(a, PH_QKV, ptarget(a, s, layer, PH_QKV), a.t_qkv, QKV, v)) return false;
        // Q scale: max over every head's rotated Q
        float mx = 0.0f;
        for (int i = tid; i < D; i += kNT) {
            const int d = i & 63;
            const float rot = d < 32 ? -v[i + 32] : v[i - 32];
            mx = fmaxf(mx, fabsf((v[i] * cs) + (rot * sn)));
        }
        mx = wave_max_f32(mx);
        if (lane == 0) misc[4 + wave] = mx;
        const float sk = a.kv_sk[layer * Hkv + gk], sv = a.kv_sv[layer * Hkv + gk];
        if (tid < 64) {
            const int i = D + gk * 64 + tid, d = tid;
            const float rot = d < 32 ? -v[i + 32] : v[i - 32];
            knew[d] = sat_i8(__builtin_rintf(__fdiv_rn((v[i] * cs) + (rot * sn), sk)));
        } else if (tid < 128) {
            const int d = tid - 64;
            vnew[d] = sat_i8(__builtin_rintf(__fdiv_rn(v[D + KVD + gk * 64 + d], sv)));
        }
        __syncthreads();
        mx = fmaxf(fmaxf(misc[4], misc[5]), fmaxf(misc[6], misc[7]));
        const double s_q = quant_scale(mx);
        const float sfq = (float)s_q;
        if (tid < 64) {
            const int i = h * 64 + tid, d = tid;
            const float rot = d < 32 ? -v[i + 32] : v[i - 32];
            qs[d] = sat_i8(__builtin_rintf(__fdiv_rn((v[i] * cs) + (rot * sn), sfq)));
        }
        if (tid == 0) misc[0] = (float)((s_q * (double)sk) * a.attn_scale);
        if (h % G == 0 && tid < 64) {
            // this step's K/V row, written through to the coherence
            // point before anything this workgroup publishes later
            __hip_atomic_store(a.kv.k + pl + KvGeom::k_off(pos, tid), knew[tid], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.kv.v + pl + KvGeom::v_off(pos, tid), vnew[tid], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0);
        }
        __syncthreads();
        // scores: lane <-> key inside a block of 64; blocks over waves
        const float scl = misc[0];
        float lmax = -INFINITY;
        for (int b0 = wave; b0 < nblk; b0 += kNW * 2) {
            v4i kk[2][4];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int8_t* kb = kp + (int64_t)min(b0 + kNW * i, nblk - 1) * 4096 + lane * 16;
#pragma unroll
                for (int q = 0; q < 4; q++) kk[i][q] = ldc16(kb + q * 1024);
            }
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int b = b0 + kNW * i, t = b * 64 + lane;
                if (b < nblk && t < T) {
                    v4i k0 = kk[i][0], k1 = kk[i][1], k2 = kk[i][2], k3 = kk[i][3];
                    if (t == pos) {
                        k0 = ((const v4i*)knew)[0];
                        k1 = ((const v4i*)knew)[1];
                        k2 = ((const v4i*)knew)[2];
                        k3 = ((const v4i*)knew)[3];
                    }
                    const v4i* q4 = (const v4i*)qs;
                    int S = sdot4v(k0, q4[0], 0);
                    S = sdot4v(k1, q4[1], S);
                    S = sdot4v(k2, q4[2], S);
                    S = sdot4v(k3, q4[3], S);
                    const float sc = (float)S * scl;
                    s_buf[t] = sc;
                    lmax = fmaxf(lmax, sc);
                }
            }
        }
        lmax = wave_max_f32(lmax);
        if (lane == 0) misc[8 + wave] = lmax;
        __syncthreads();
        if (tid == 0) misc[1] = fmaxf(fmaxf(misc[8], misc[9]), fmaxf(misc[10], misc[11]));
        __syncthreads();
        const float mrow = misc[1];
        for (int b = wave; b < nblk; b += kNW) {
            const int t = b * 64 + lane;
            float e = 0.0f;
            if (t < T) {
                e = tl_expf(s_buf[t] - mrow);
                s_buf[t] = e;
            }
            const float bs = wave_butterfly_sum(e);
            if (lane == 0) bsum[b] = bs;
        }
        __syncthreads();
        if (tid == 0) {
            float total = 0.0f;
            for (int b = 0; b < nblk; b++) total = total + bsum[b];
            misc[2] = total;
        }
        __syncthreads();
        const float tot = misc[2];
        for (int t = tid; t < tpad; t += kNT) {
            int8_t pq = 0;
            if (t < T) {
                float pr = __builtin_rintf(__fdiv_rn(s_buf[t], tot) * 127.0f);
                pr = pr < 0.0f ? 0.0f : (pr > 127.0f ? 127.0f : pr);
                pq = (int8_t)(int)pr;
            }
            p8[t] = pq;
        }
        __syncthreads();
        // O = P8 . V8, lane <-> dimension; this step's V row from vnew
        int o = 0;
        const int cpos = pos >> 4, bpos = pos & 15;
        for (int c0 = wave; c0 < ngrp; c0 += kNW * 4) {
            v4i vv[4];
#pragma unroll
            for (int j = 0; j < 4; j++) vv[j] = ldc16(vp + (int64_t)min(c0 + kNW * j, ngrp - 1) * 1024 + lane * 16);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int c = c0 + kNW * j;
                if (c < ngrp) {
                    v4i x = vv[j];
                    if (c == cpos) {
                        const unsigned nb = (uint8_t)vnew[lane];
                        const int sh = (bpos & 3) * 8;
                        const unsigned keep = ~(0xFFu << sh);
                        const int q = bpos >> 2;
                        x[q] = (int)(((unsigned)x[q] & keep) | (nb << sh));
                    }
                    o = sdot4v(x, *(const v4i*)(p8 + c * 16), o);
                }
            }
        }
        accs[wave * 64 + lane] = o;
        __syncthreads();
        if (tid < 64) {
            const int O = accs[tid] + accs[64 + tid] + accs[128 + tid] + accs[192 + tid];
            putf(a.t_att + h * 64 + tid, (float)O * deq_mult(1.0 / 127.0, sv));
        }
        signal_phase(a.ctr, PH_ATT);
    }
    return true;
}

// P3 + P4: attended -> O rows + residual, then RMSNorm -> gate/up rows ->
// SiLU-GLU.  Both weight sets are requested on entry, so the gate/up stream
// runs while the attention phase and the O phase are awaited.
template <int KD>
__device__ __noinline__ bool ph_o_glu(KArgs* ap, int s, int layer, int tok) {
    KArgs& a = uniform_args(ap);
    s = __builtin_amdgcn_readfirstlane(s);
    layer = __builtin_amdgcn_readfirstlane(layer);
    tok = __builtin_amdgcn_readfirstlane(tok);
    const Lds L = lds_map();
    const int lane = threadIdx.x & 63;
    const int D = a.D, F = a.F;
    KLayer& Ly = klayer(a, layer);
    constexpr int RO = 3, RG = 8;
    GemvPhase go{Ly.wo, nullptr, Ly.so, nullptr, D, D};
    GemvPhase gg{Ly.wg, Ly.wu, Ly.sg, Ly.su, F, D};
    // the weights, then the residual rows (complete since this workgroup's
    // P1 waited for them); wavefront 0 loads neither
    int ro = first_row(RO), rg = first_row(RG);
    auto residual = [&](int r) {   // the layer's input x at row r + lane (layer 0: the embedding row)
        const int n = r + lane;
        if (r >= D || lane >= RO || n >= D) return 0.0f;
        return layer == 0 ? (float)a.emb[(int64_t)tok * D + n] * a.emb_s[tok] : getf(a.t_x + n);
    };
    v4i wo[1][RO][KD];
    v4i wg[2][RG][KD];
    if (ro < D) load_rows<1, RO, KD>(go, ro, wo);
    if (rg < F) load_rows<2, RG, KD>(gg, rg, wg);
    float res = residual(ro);

    // P3
    if (!wait_stage<KD * 4>(a, PH_ATT, ptarget(a, s, layer, PH_ATT), a.t_att, D, L.att)) return false;
    {
        float4 xv[KD];
        chunks_from<KD>(L.att, D, xv);
        prologue_quant<KD>(xv, D, L.xs8, L.red, L.xscale);
    }
    double sx = *L.xscale;
    for (; ro < D; ro += row_stride(RO)) {
        if (ro != first_row(RO)) {
            load_rows<1, RO, KD>(go, ro, wo);
            res = residual(ro);
        }
        int mine[1];
        dot_rows<1, RO, KD>(wo, L.xs8, D, mine);
        const int n = ro + lane;
        if (lane < RO && n < D) putf(a.t_xa + n, res + (float)mine[0] * deq_mult(sx, go.ws[n]));
    }
    signal_phase(a.ctr, PH_O);

    // P4
    if (!wait_stage<KD * 4>(a, PH_O, ptarget(a, s, layer, PH_O), a.t_xa, D, L.att)) return false;
    {
        float4 xv[KD], gv[KD];
        chunks_from<KD>(L.att, D, xv);
        gamma_chunks<KD>(Ly.g_post, D, gv);
        prologue_rmsnorm<KD>(xv, gv, D, a.eps, PwPlan{a.plan.leaf_len, a.plan.n_leaves}, L.sq, L.part, L.xs8, L.red, L.xscale);
    }
    sx = *L.xscale;
    for (; rg < F; rg += row_stride(RG)) {
        if (rg != first_row(RG)) load_rows<2, RG, KD>(gg, rg, wg);
        int mine[2];
        dot_rows<2, RG, KD>(wg, L.xs8, D, mine);
        const int n = rg + lane;
        if (lane < RG && n < F) {
            const float gt = (float)mine[0] * deq_mult(sx, gg.ws[n]);
            const float up = (float)mine[1] * deq_mult(sx, gg.ws2[n]);
            putf(a.t_h + n, tl_silu(gt) * up);
        }
    }
    signal_phase(a.ctr, PH_GLU);
    return true;
}

// P5 + the next layer's P1: hidden -> down rows + residual -> x, then
// RMSNorm -> Q|K|V rows of layer + 1 (skipped after the last layer)
template <int KD, int KF>
__device__ __noinline__ bool ph_down_qkv(KArgs* ap, int s, int layer) {
    KArgs& a = uniform_args(ap);
    s = __builtin_amdgcn_readfirstlane(s);
    layer = __builtin_amdgcn_readfirstlane(layer);
    const Lds L = lds_map();
    const int lane = threadIdx.x & 63;
    const int D = a.D, F = a.F, QKV = D + 2 * a.Hkv * kHeadDim;
    KLayer& Ly = klayer(a, layer);
    const bool next = layer + 1 < a.n_layers;
    constexpr int RD = 3, RQ = 4;
    GemvPhase gd{Ly.wd, nullptr, Ly.sd, nullptr, D, F};
    GemvPhase gq{next ? klayer(a, layer + 1).wqkv : Ly.wqkv, nullptr, next ? klayer(a, layer + 1).sqkv : Ly.sqkv,
                 nullptr, QKV, D};
    // the weights, then the residual rows (complete since the P4 wait)
    int rd = first_row(RD), rq = first_row(RQ);
    v4i wd[1][RD][KF];
    v4i wq[1][RQ][KD];
    if (rd < D) load_rows<1, RD, KF>(gd, rd, wd);
    if (next && rq < QKV) load_rows<1, RQ, KD>(gq, rq, wq);
    float res = 0.0f;
    if (rd < D && lane < RD && rd + lane < D) res = getf(a.t_xa + rd + lane);

    // P5
    if (!wait_stage<KF * 4>(a, PH_GLU, ptarget(a, s, layer, PH_GLU), a.t_h, F, L.att)) return false;
    {
        float4 xv[KF];
        chunks_from<KF>(L.att, F, xv);
        prologue_quant<KF>(xv, F, L.xs8, L.red, L.xscale);
    }
    double sx = *L.xscale;
    for (; rd < D; rd += row_stride(RD)) {
        if (rd != first_row(RD)) {
            load_rows<1, RD, KF>(gd, rd, wd);
            if (lane < RD && rd + lane < D) res = getf(a.t_xa + rd + lane);
        }
        int mine[1];
        dot_rows<1, RD, KF>(wd, L.xs8, F, mine);
        const int n = rd + lane;
        if (lane < RD && n < D) putf(a.t_x + n, res + (float)mine[0] * deq_mult(sx, gd.ws[n]));
    }
    signal_phase(a.ctr, PH_DOWN);
    if (!next) return true;

    // P1 of layer + 1
    KLayer& Ln = klayer(a, layer + 1);
    if (!wait_stage<KD * 4>(a, PH_DOWN, ptarget(a, s, layer, PH_DOWN), a.t_x, D, L.att)) return false;
    {
        float4 xv[KD], gv[KD];
        chunks_from<KD>(L.att, D, xv);
        gamma_chunks<KD>(Ln.g_in, D, gv);
        prologue_rmsnorm<KD>(xv, gv, D, a.eps, PwPlan{a.plan.leaf_len, a.plan.n_leaves}, L.sq, L.part, L.xs8, L.red, L.xscale);
    }
    sx = *L.xscale;
    for (; rq < QKV; rq += row_stride(RQ)) {
        if (rq != first_row(RQ)) load_rows<1, RQ, KD>(gq, rq, wq);
        int mine[1];
        dot_rows<1, RQ, KD>(wq, L.xs8, D, mine);
        const int n = rq + lane;
        if (lane < RQ && n < QKV) putf(a.t_qkv + n, (float)mine[0] * deq_mult(sx, gq.ws[n]));
    }
    signal_phase(a.ctr, PH_QKV);
    return true;
}

// P6: final RMSNorm -> LM head rows -> this workgroup's best key folded into
// the step's key, then the workgroup is counted in
template <int KD>
__device__ __noinline__ bool ph_lm(KArgs* ap, int s) {
    KArgs& a = uniform_args(ap);
    s = __builtin_amdgcn_readfirstlane(s);
    const Lds L = lds_map();
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int D = a.D;
    constexpr int RB = 8;
    GemvPhase g{a.lm_w, nullptr, a.lm_s, nullptr, a.V, D};
    v4i wv[1][RB][KD];
    int r0 = first_row(RB);
    if (r0 < a.V) load_rows<1, RB, KD>(g, r0, wv);
    if (!wait_stage<KD * 4>(a, PH_DOWN, ptarget(a, s, a.n_layers - 1, PH_DOWN), a.t_x, D, L.att)) return false;
    {
        float4 xv[KD], gv[KD];
        chunks_from<KD>(L.att, D, xv);
        gamma_chunks<KD>(a.g_final, D, gv);
        prologue_rmsnorm<KD>(xv, gv, D, a.eps, PwPlan{a.plan.leaf_len, a.plan.n_leaves}, L.sq, L.part, L.xs8, L.red, L.xscale);
    }
    const double sx = *L.xscale;
    unsigned long long best = 0;
    for (; r0 < a.V; r0 += row_stride(RB)) {
        if (r0 != first_row(RB)) load_rows<1, RB, KD>(g, r0, wv);
        int mine[1];
        dot_rows<1, RB, KD>(wv, L.xs8, D, mine);
        const int n = r0 + lane;
        if (lane < RB && n < a.V) {
            const unsigned long long k = argmax_key((float)mine[0] * deq_mult(sx, g.ws[n]), n);
            best = k > best ? k : best;
        }
    }
    best = wave_max_u64(best);
    if (lane == 0) L.wbest[wave] = best;
    __syncthreads();
    if (tid == 0) {
        unsigned long long b = L.wbest[0];
        for (int i = 1; i < kNW; i++) b = L.wbest[i] > b ? L.wbest[i] : b;
        __hip_atomic_fetch_max(a.keys + s, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);   // the max is complete before the count
        __hip_atomic_fetch_add(a.done + s, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return true;
}

template <int KD, int KF>
__global__ __launch_bounds__(kNT) void persist_decode_kernel(PersistArgs) {
    KArgs* ap = (KArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    KArgs& a = *ap;
    const Lds L = lds_map();
    const int tid = threadIdx.x;
    const int nwg = gridDim.x, wg = blockIdx.x;
    unsigned* err = a.err;
    int tok = min(max(a.token_cur[a.seq], 0), a.V - 1);
    const int pos0 = a.cursor[a.seq];
    const int ngen0 = a.n_gen[a.seq];
    int steps = 0;

    for (int s = 0; s < a.n_steps; s++) {
        const int pos = pos0 + s;
        if (!ph_qkv0<KD>(ap, s, tok)) return;
        for (int layer = 0; layer < a.n_layers; layer++) {
            if (wg < a.H && !ph_att(ap, s, layer, pos)) return;
            if (!ph_o_glu<KD>(ap, s, layer, tok)) return;
            if (!ph_down_qkv<KD, KF>(ap, s, layer)) return;
        }
        if (!ph_lm<KD>(ap, s)) return;
        // ---- the step's token, seen by every workgroup ---------------------------
        {
            if (tid == 0) {
                unsigned it = 0;
                bool ok = true;
                while (peek32(a.done + s) < (unsigned)nwg) {
                    if ((it & 63) == 63 && peek32(err)) { ok = false; break; }
                    if (++it > kSpinLimit) {
                        __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        ok = false;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                const unsigned long long k =
                    ok ? __hip_atomic_load(a.keys + s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
                L.wbest[0] = ok ? k : ~0ull;
            }
            __syncthreads();
            const unsigned long long k = L.wbest[0];
            if (k == ~0ull) return;
            tok = min(max(key_index(k), 0), a.V - 1);
            steps = s + 1;
            if (wg == 0 && tid == 0) {
                const int i = ngen0 + s;
                if (i >= 0 && i < a.out_stride) {
                    a.tokens_out[(int64_t)a.seq * a.out_stride + i] = tok;
                    a.logit_out[(int64_t)a.seq * a.out_stride + i] = key_logit(k);
                }
            }
            __syncthreads();
            if (a.eos_id >= 0 && tok == a.eos_id) break;
        }
    }
    if (wg == 0 && tid == 0) {
        a.token_cur[a.seq] = tok;
        a.n_gen[a.seq] = ngen0 + steps;
        a.cursor[a.seq] = pos0 + steps;
        a.status[0] = steps;
    }
}

size_t persist_lds_bytes(int32_t qkv, int32_t f, int32_t max_pos) {
    const size_t tpad = ((size_t)max_pos + 63) & ~(size_t)63;
    const size_t att = sizeof(float) * qkv + tpad * 4 + tpad + ((tpad / 64 + 3) & ~(size_t)3) * 4 + 3 * 64 + 16 * 4 +
                       4 * 64 * 4;
    const size_t stage = sizeof(float) * (((size_t)std::max(f, qkv) + 255) & ~(size_t)255);   // staged inputs, whole slices
    return 6144 + 8192 + 2048 + 256 + ((std::max(att, stage) + 15) & ~(size_t)15);
}

bool persist_supported(int32_t d, int32_t f, int32_t qkv) {
    const int kd = (d + 1023) / 1024, kf = (f + 1023) / 1024;
    if (qkv > kQkvPerThread * kNT) return false;
    return (kd == 2 && kf == 6) || (kd == 1 && kf == 2) || (kd == 1 && kf == 1) || (kd == 2 && kf == 2);
}

static const void* persist_fn(int32_t d, int32_t f) {
    const int kd = (d + 1023) / 1024, kf = (f + 1023) / 1024;
    if (kd == 2 && kf == 6) return (const void*)persist_decode_kernel<2, 6>;
    if (kd == 1 && kf == 2) return (const void*)persist_decode_kernel<1, 2>;
    if (kd == 1 && kf == 1) return (const void*)persist_decode_kernel<1, 1>;
    if (kd == 2 && kf == 2) return (const void*)persist_decode_kernel<2, 2>;
    return nullptr;
}

hipError_t persist_occupancy(int32_t d, int32_t f, size_t lds, int* blocks_per_cu) {
    const void* fn = persist_fn(d, f);
    if (!fn) return hipErrorInvalidValue;
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, fn, kNT, lds);
}

hipError_t launch_persist_decode(hipStream_t s, const PersistArgs& args, int32_t grid, size_t lds) {
    const void* fn = persist_fn(args.D, args.F);
    if (!fn) return hipErrorInvalidValue;
    PersistArgs copy = args;
    void* kargs[] = {&copy};
    return hipLaunchCooperativeKernel(fn, dim3(grid), dim3(kNT), kargs, (unsigned)lds, s);
}

}  // namespace tl
