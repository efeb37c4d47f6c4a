// tl_decode.hip -- fused kernels of the batch-1 decode step (five kernels per
// decoder layer, each ending at one of the global reductions the reference's
// per-tensor activation quantization requires):
//
//   gemv_fused<RMSNORM, DEQUANT>   x -> RMSNorm -> INT8 -> Q|K|V projections
//   attention_decode               RoPE, Q to INT8, K/V to the cache, GQA attention
//   gemv_fused<QUANT, DEQUANT_RES> attended -> INT8 -> O projection + residual
//   gemv_fused<RMSNORM, GLU>       x -> RMSNorm -> INT8 -> gate/up -> SiLU(gate)*up
//   gemv_fused<QUANT, DEQUANT_RES> hidden -> INT8 -> down projection + residual
//
// Every workgroup of a fused GEMV first issues the global loads of its
// activation row, then all of its weight rows (one 128-bit load per lane per
// KiB of row), and only then runs the prologue (RMSNorm / quantization of the
// activation into LDS), so the weight stream is in flight while the prologue
// computes.  The prologue is the same arithmetic as the standalone kernels
// (NumPy pairwise tree for the sum of squares, float64 scale), so results are
// bit-identical to them and to the CPU oracle.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "tl_device.h"
#include "tl_internal.h"
#include "tl_prologue.h"

namespace tl {

// ---------------------------------------------------------------------------
// fused decode GEMV: y = epilogue(W . prologue(x)); 4 wavefronts x R rows
// ---------------------------------------------------------------------------
template <int PRO, int EPI, int R, int KCH>
__global__ __launch_bounds__(kNT) void gemv_fused_kernel(GemvArgs a) {
    constexpr int NM = (EPI == EPI_GLU) ? 2 : 1;
    __shared__ __align__(16) int8_t xs8[KCH * 1024];
    __shared__ __align__(16) float sq[PRO == PRO_RMSNORM ? KCH * 1024 : 4];
    __shared__ __align__(16) float part[PRO == PRO_RMSNORM ? 8 * 64 : 4];
    __shared__ float red[16];
    __shared__ double xscale;
    __shared__ unsigned long long wbest[kNW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const WaveStamp stamp(a.ts, (int64_t)blockIdx.x * kNW + wave);
    const int K = a.k;
    const int row0 = (blockIdx.x * kNW + wave) * R;

    // 1) activation row and this lane's epilogue operands first (clamped
    // indices, no branches): lane l < R finishes row row0 + l ...
    float4 xv[KCH], gv[KCH];
    v4i xr[KCH];
    const int kq = K / 4 - 1;
    const int nl = min(row0 + min(lane, R - 1), a.n - 1);
    const float wsl = a.ws[nl];
    const float ws2l = (EPI == EPI_GLU) ? a.ws2[nl] : 0.0f;
    const float resl = (EPI == EPI_DEQUANT_RES) ? a.residual[nl] : 0.0f;
    if (PRO == PRO_X8) {
#pragma unroll
        for (int c = 0; c < KCH; c++) {
            const int off = c * 1024 + lane * 16;
            xr[c] = ld16(a.x + min(off, K - 16));
        }
    } else {
#pragma unroll
        for (int c = 0; c < KCH; c++) {
            const int idx = min(c * kNT + tid, kq);
            xv[c] = ((const float4*)a.xf)[idx];
            if (PRO == PRO_RMSNORM) gv[c] = ((const float4*)a.gamma)[idx];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // 2) ... then every weight row of this wavefront: unconditional 128-bit
    // non-temporal loads; lanes past the end of a row read an in-bounds
    // stand-in and meet zero activation bytes
    v4i wv[NM][R][KCH];
#pragma unroll
    for (int m = 0; m < NM; m++) {
        const int8_t* wb = m ? a.w2 : a.w;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int8_t* wr = wb + (int64_t)min(row0 + r, a.n - 1) * K;
#pragma unroll
            for (int c = 0; c < KCH; c++) wv[m][r][c] = ld_nt16(wr + min(c * 1024 + lane * 16, K - 16));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // 3) prologue while the weights stream in
    double sx;
    if (PRO == PRO_X8) {
        sx = a.xs[0];
#pragma unroll
        for (int c = 0; c < KCH; c++)
            if (c * 1024 + lane * 16 >= K) xr[c] = (v4i){0, 0, 0, 0};
    } else {
        if (PRO == PRO_QUANT) prologue_quant<KCH>(xv, K, xs8, red, &xscale);
        else prologue_rmsnorm<KCH>(xv, gv, K, a.eps, a.plan, sq, part, xs8, red, &xscale);
        sx = xscale;
#pragma unroll
        for (int c = 0; c < KCH; c++) xr[c] = ld16(xs8 + c * 1024 + lane * 16);
    }
    // 4) dot products and wavefront reductions (exact integers)
    int acc[NM][R];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int r = 0; r < R; r++) {
            int s = 0;
#pragma unroll
            for (int c = 0; c < KCH; c++) s = sdot4v(wv[m][r][c], xr[c], s);
            acc[m][r] = wave_sum_i32(s);
        }
    // 5) epilogue: the sums are wavefront-uniform; lane l < R takes row l's
    int mine[NM];
#pragma unroll
    for (int m = 0; m < NM; m++) {
        mine[m] = acc[m][0];
#pragma unroll
        for (int r = 1; r < R; r++) mine[m] = lane == r ? acc[m][r] : mine[m];
    }
    const int n = row0 + lane;
    const bool live = lane < R && n < a.n;
    if (EPI == EPI_ARGMAX) {
        unsigned long long k = 0;
        if (live) {
            const float logit = (float)mine[0] * deq_mult(sx, wsl);
            if (a.y) a.y[n] = logit;
            k = argmax_key(logit, n);
        }
        const unsigned long long best = wave_max_u64(k);
        if (lane == 0) wbest[wave] = best;
        __syncthreads();
        if (tid == 0) {
            unsigned long long b = wbest[0];
            for (int i = 1; i < kNW; i++) b = wbest[i] > b ? wbest[i] : b;
            if (a.wg_keys) a.wg_keys[blockIdx.x] = b;   // folded by the consumer
            else if (b) atomicMax(a.key, b);
        }
        return;
    }
    if (!live) return;
    if (EPI == EPI_DEQUANT || EPI == EPI_DEQUANT_RES) {
        float v = (float)mine[0] * deq_mult(sx, wsl);
        if (EPI == EPI_DEQUANT_RES) v = resl + v;
        a.y[n] = v;
    } else if (EPI == EPI_GLU) {
        const float gt = (float)mine[0] * deq_mult(sx, wsl);
        const float up = (float)mine[NM - 1] * deq_mult(sx, ws2l);
        a.y[n] = tl_silu(gt) * up;
    }
}

// ---------------------------------------------------------------------------
// decode attention with the Q/K/V post-processing fused in.  One workgroup
// per (row, HPW query heads); for query position pos the keys are 0..pos, of
// which 0..pos-1 are read from the cache and pos is this step's own row,
// computed here: RoPE (TL:69-80) on Q and K, Q quantized at the row's scale
// (max over all heads), K and V at the static per-layer/per-KV-head scales.
// The first workgroup of each KV head writes that row to the cache.
// ---------------------------------------------------------------------------
struct AttnDecodeArgs {
    const float* qkv;     // [rows][D + 2 KVD]
    int32_t n_heads, n_kv;
    RowMap rm;
    const float* cosb;
    const float* sinb;
    KvGeom kv;
    int32_t layer;
    const float* kv_sk;
    const float* kv_sv;
    double attn_scale;
    float* out;           // [rows][D]
    unsigned long long* ts;   // decode timeline: [waves][2] clock stamps, or null
    // the grouped kernel may read Q|K|V as the integer sums of a K-sliced GEMM
    // instead (qkv unused): value i of a row = f32(qacc[i]) f32(qas[row] qws[i]),
    // the GEMM's DEQUANT epilogue
    const int32_t* qacc;  // [rows][D + 2 KVD] or null
    const double* qas;    // [rows]
    const float* qws;     // [D + 2 KVD]
    float* out_max;       // attention_group_kernel: [rows][n_heads] max |output| of each head, or null
};

// NW wavefronts per workgroup; wavefront w takes key blocks w, w + NW, ...
// (and value groups likewise).  Past the KPF / VPF blocks prefetched during
// the Q/K/V post-processing, each wavefront loads KB key blocks (VB value
// groups) before it computes any of them, so one memory latency covers
// several blocks.
template <int HPW, int KPF, int VPF, int NW>
__global__ __launch_bounds__(NW * 64) void attention_decode_kernel(AttnDecodeArgs p) {
    constexpr int NT = NW * 64, KB = HPW > 1 ? 2 : 4, VB = HPW > 1 ? 4 : 8;
    extern __shared__ __align__(16) float dyn[];
    __shared__ __align__(16) int8_t qs[HPW][64];
    __shared__ __align__(16) int8_t knew[64];
    __shared__ __align__(16) int8_t vnew[64];
    __shared__ float red[NW];
    __shared__ float scl[HPW], mrow[HPW], tot[HPW];
    __shared__ float wmax[NW][HPW];
    __shared__ int accs[NW][HPW][64];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = p.n_heads / p.n_kv;
    int hb = blockIdx.x;
    if (HPW == 1 && p.n_heads == 32 && p.n_kv == 4) {
        // keep the 8 query heads of a KV head on two XCDs (workgroups are
        // dispatched round-robin over the 8 XCDs) so its K/V rows are shared
        // through their L2 caches
        const int xcd = hb & 7, slot = hb >> 3;
        hb = (xcd >> 1) * 8 + (xcd & 1) * 4 + slot;
    }
    const int h0 = hb * HPW;
    const int g = h0 / G;
    const int row = blockIdx.y;
    const int D = p.n_heads * kHeadDim, KVD = p.n_kv * kHeadDim, W = D + 2 * KVD;
    const int pos = p.rm.pos[row], seq = p.rm.seq[row];
    if (pos < 0 || pos >= p.kv.max_pos) return;   // a row outside the cache (uniform per workgroup)
    const int T = pos + 1;
    const int tpad = (T + 63) & ~63;
    const int nblk = tpad >> 6;
    const int ngrp = tpad >> 4;
    const int64_t pl = p.kv.plane(seq, p.layer, g);
    const int8_t* kp = p.kv.k + pl;
    const int8_t* vp = p.kv.v + pl;

    float* v = dyn;                          // [W] this row's q|k|v
    float* s_buf = dyn + W;                  // [HPW][tpad] scores, then exps
    int8_t* p8 = (int8_t*)(s_buf + HPW * tpad);
    float* bsum = (float*)(p8 + HPW * tpad); // [HPW][nblk]

    // 0) this row's q|k|v into LDS (just written by the projection kernel,
    //    an L2 hit) ...
    const float* src = p.qkv + (int64_t)row * W;
    // every element a thread rotates has dimension tid % 64 (NT = NW x 64)
    const float cs = p.cosb[(int64_t)pos * kHeadDim + (tid & 63)];
    const float sn = p.sinb[(int64_t)pos * kHeadDim + (tid & 63)];
    for (int i = tid; i < W / 4; i += NT) ((float4*)v)[i] = ((const float4*)src)[i];
    __syncthreads();
    // ... then the cached K/V rows this wavefront will use (rows 0..pos-1 are
    //    final), in flight during the RoPE / quantization below; block and
    //    group indices are clamped so the loads stay inside the plane and the
    //    surplus copies are never used
    v4i kreg[KPF][4], vreg[VPF];
#pragma unroll
    for (int i = 0; i < KPF; i++) {
        const int8_t* kb = kp + (int64_t)min(wave + NW * i, nblk - 1) * 4096 + lane * 16;
#pragma unroll
        for (int q = 0; q < 4; q++) kreg[i][q] = ld16(kb + q * 1024);
    }
#pragma unroll
    for (int j = 0; j < VPF; j++) vreg[j] = ld16(vp + (int64_t)min(wave + NW * j, ngrp - 1) * 1024 + lane * 16);
    __builtin_amdgcn_sched_barrier(0);

    // RoPE of every Q element (the row's scale is the max over all heads)
    float mx = 0.0f;
    for (int i = tid; i < D; i += NT) {
        const int d = i & 63;
        const float rot = d < 32 ? -v[i + 32] : v[i - 32];
        mx = fmaxf(mx, fabsf((v[i] * cs) + (rot * sn)));
    }
    mx = wave_max_f32(mx);
    if (lane == 0) red[wave] = mx;
    // this row's K (after RoPE) and V of KV head g at the static scales
    const float sk = p.kv_sk[p.layer * p.n_kv + g], sv = p.kv_sv[p.layer * p.n_kv + g];
    if (tid < 64) {
        const int i = D + g * 64 + tid, d = tid;
        const float rot = d < 32 ? -v[i + 32] : v[i - 32];
        const float kr = (v[i] * cs) + (rot * sn);
        knew[d] = sat_i8(__builtin_rintf(__fdiv_rn(kr, sk)));
    } else if (tid < 128) {
        const int d = tid - 64;
        vnew[d] = sat_i8(__builtin_rintf(__fdiv_rn(v[D + KVD + g * 64 + d], sv)));
    }
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < NW; w++) mx = fmaxf(mx, red[w]);
    const double s_q = quant_scale(mx);
    const float sfq = (float)s_q;
    for (int e = tid; e < HPW * 64; e += NT) {   // e % 64 == tid % 64: cs, sn apply
        const int i = h0 * 64 + e, d = e & 63;
        const float rot = d < 32 ? -v[i + 32] : v[i - 32];
        qs[e >> 6][d] = sat_i8(__builtin_rintf(__fdiv_rn((v[i] * cs) + (rot * sn), sfq)));
    }
    if (tid < HPW) scl[tid] = (float)((s_q * (double)sk) * p.attn_scale);
    if (h0 % G == 0 && tid < 64) {
        p.kv.k[pl + KvGeom::k_off(pos, tid)] = knew[tid];
        p.kv.v[pl + KvGeom::v_off(pos, tid)] = vnew[tid];
    }
    __syncthreads();

    // scores: lane <-> key inside a block of 64
    float lmax[HPW];
#pragma unroll
    for (int h = 0; h < HPW; h++) lmax[h] = -INFINITY;
    auto score_block = [&](int b, v4i k0, v4i k1, v4i k2, v4i k3) {
        const int t = b * 64 + lane;
        if (t < T) {
            if (t == pos) {
                k0 = ((const v4i*)knew)[0];
                k1 = ((const v4i*)knew)[1];
                k2 = ((const v4i*)knew)[2];
                k3 = ((const v4i*)knew)[3];
            }
#pragma unroll
            for (int h = 0; h < HPW; h++) {
                const v4i* q4 = (const v4i*)qs[h];
                int S = sdot4v(k0, q4[0], 0);
                S = sdot4v(k1, q4[1], S);
                S = sdot4v(k2, q4[2], S);
                S = sdot4v(k3, q4[3], S);
                const float sv2 = (float)S * scl[h];
                s_buf[h * tpad + t] = sv2;
                lmax[h] = fmaxf(lmax[h], sv2);
            }
        }
    };
#pragma unroll
    for (int i = 0; i < KPF; i++)
        if (wave + NW * i < nblk) score_block(wave + NW * i, kreg[i][0], kreg[i][1], kreg[i][2], kreg[i][3]);
    for (int b0 = wave + NW * KPF; b0 < nblk; b0 += NW * KB) {
        v4i kk[KB][4];
#pragma unroll
        for (int i = 0; i < KB; i++) {
            const int8_t* kb = kp + (int64_t)min(b0 + NW * i, nblk - 1) * 4096 + lane * 16;
#pragma unroll
            for (int q = 0; q < 4; q++) kk[i][q] = ld16(kb + q * 1024);
        }
#pragma unroll
        for (int i = 0; i < KB; i++)
            if (b0 + NW * i < nblk) score_block(b0 + NW * i, kk[i][0], kk[i][1], kk[i][2], kk[i][3]);
    }
#pragma unroll
    for (int h = 0; h < HPW; h++) {
        const float m = wave_max_f32(lmax[h]);
        if (lane == 0) wmax[wave][h] = m;
    }
    __syncthreads();
    if (tid < HPW) {
        float m = wmax[0][tid];
        for (int w = 1; w < NW; w++) m = fmaxf(m, wmax[w][tid]);
        mrow[tid] = m;
    }
    __syncthreads();
    // exponentials and the block-64 butterfly sums
    for (int b = wave; b < nblk; b += NW) {
        const int t = b * 64 + lane;
#pragma unroll
        for (int h = 0; h < HPW; h++) {
            float e = 0.0f;
            if (t < T) {
                e = tl_expf(s_buf[h * tpad + t] - mrow[h]);
                s_buf[h * tpad + t] = e;
            }
            const float bs = wave_butterfly_sum(e);
            if (lane == 0) bsum[h * nblk + b] = bs;
        }
    }
    __syncthreads();
    if (tid < HPW) {
        float total = 0.0f;
        for (int b = 0; b < nblk; b++) total = total + bsum[tid * nblk + b];
        tot[tid] = total;
    }
    __syncthreads();
    for (int t = tid; t < tpad; t += blockDim.x) {
#pragma unroll
        for (int h = 0; h < HPW; h++) {
            int8_t pq = 0;
            if (t < T) {
                float pr = __builtin_rintf(__fdiv_rn(s_buf[h * tpad + t], tot[h]) * 127.0f);
                pr = pr < 0.0f ? 0.0f : (pr > 127.0f ? 127.0f : pr);
                pq = (int8_t)(int)pr;
            }
            p8[h * tpad + t] = pq;
        }
    }
    __syncthreads();
    // O = P8 . V8, lane <-> dimension; this row's V comes from vnew
    int o[HPW];
#pragma unroll
    for (int h = 0; h < HPW; h++) o[h] = 0;
    const int cpos = pos >> 4, bpos = pos & 15;
    auto pv_group = [&](int c, v4i vv) {
        if (c == cpos) {
            const unsigned nb = (uint8_t)vnew[lane];
            const int sh = (bpos & 3) * 8;
            const unsigned keep = ~(0xFFu << sh);
            const int q = bpos >> 2;
            vv[q] = (int)(((unsigned)vv[q] & keep) | (nb << sh));
        }
#pragma unroll
        for (int h = 0; h < HPW; h++) o[h] = sdot4v(vv, *(const v4i*)(p8 + h * tpad + c * 16), o[h]);
    };
#pragma unroll
    for (int j = 0; j < VPF; j++)
        if (wave + NW * j < ngrp) pv_group(wave + NW * j, vreg[j]);
    for (int c0 = wave + NW * VPF; c0 < ngrp; c0 += NW * VB) {
        v4i vv[VB];
#pragma unroll
        for (int j = 0; j < VB; j++) vv[j] = ld16(vp + (int64_t)min(c0 + NW * j, ngrp - 1) * 1024 + lane * 16);
#pragma unroll
        for (int j = 0; j < VB; j++)
            if (c0 + NW * j < ngrp) pv_group(c0 + NW * j, vv[j]);
    }
#pragma unroll
    for (int h = 0; h < HPW; h++) accs[wave][h][lane] = o[h];
    __syncthreads();
    const float pv_mult = deq_mult(1.0 / 127.0, sv);
    for (int i = tid; i < HPW * 64; i += blockDim.x) {
        const int h = i >> 6, d = i & 63;
        int O = 0;
#pragma unroll
        for (int w = 0; w < NW; w++) O += accs[w][h][d];
        p.out[(int64_t)row * D + (int64_t)(h0 + h) * kHeadDim + d] = (float)O * pv_mult;
    }
}

// ---------------------------------------------------------------------------
// decode attention, one workgroup (4 wavefronts) per (row, query head), same
// arithmetic as attention_decode_kernel<1, ...>.  Wavefront w owns the key
// blocks b = w + 4 i (64 keys each) for scores, exponentials, probabilities
// and P.V (the V groups 4 b .. 4 b + 3 are the same keys), so only the row's
// Q scale, the score maximum, the block sums and the output cross
// wavefronts: four barriers.  The K/V rows of the first KPF blocks are
// requested right after the few Q/K/V values this workgroup needs, before
// any of them is awaited.  Every wavefront keeps its own copy of the head's
// INT8 Q and of this row's INT8 K (lane d <-> dimension d; RoPE's partner
// dimension d ^ 32 is lane d ^ 32 of the same wavefront).
// ---------------------------------------------------------------------------
constexpr int kRowQPerThread = 16;   // Q width <= 16 x 256

template <int KPF>
__global__ __launch_bounds__(256) void attention_row_kernel(AttnDecodeArgs p) {
    constexpr int NW = 4, KB = 4;
    extern __shared__ __align__(16) float dyn[];
    __shared__ __align__(16) int8_t qs[NW][64];
    __shared__ __align__(16) int8_t kn[NW][64];
    __shared__ float red[NW], wmax[NW];
    __shared__ int accs[NW][64];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const WaveStamp stamp(p.ts, ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * NW + wave);
    const int G = p.n_heads / p.n_kv;
    int h0 = blockIdx.x;
    if (p.n_heads == 32 && p.n_kv == 4) {
        // the 8 query heads of a KV head on two XCDs (workgroups go round-robin
        // over the 8 XCDs), so its K/V rows are shared through their L2 caches
        const int xcd = h0 & 7, slot = h0 >> 3;
        h0 = (xcd >> 1) * 8 + (xcd & 1) * 4 + slot;
    }
    const int g = h0 / G, row = blockIdx.y;
    const int D = p.n_heads * kHeadDim, KVD = p.n_kv * kHeadDim, W = D + 2 * KVD;
    const int pos = p.rm.pos[row], seq = p.rm.seq[row];
    if (pos < 0 || pos >= p.kv.max_pos) return;   // a row outside the cache (uniform per workgroup)
    const int T = pos + 1, tpad = (T + 63) & ~63, nblk = tpad >> 6;
    const int64_t pl = p.kv.plane(seq, p.layer, g);
    const int8_t* kp = p.kv.k + pl;
    const int8_t* vp = p.kv.v + pl;
    float* s_buf = dyn;                          // [tpad] scores, then exponentials
    int8_t* p8 = (int8_t*)(dyn + tpad);          // [tpad]
    float* bsum = (float*)(p8 + tpad);           // [nblk]
    const float* src = p.qkv + (int64_t)row * W;
    const int d = lane;

    // 1) RoPE factors, every Q element (the row's scale is the max over all
    //    heads; element tid + 256 j has dimension d), this head's Q, this
    //    row's K and V (clamped, in-bounds indices) ...
    const float cs = p.cosb[(int64_t)pos * kHeadDim + d];
    const float sn = p.sinb[(int64_t)pos * kHeadDim + d];
    const int nq = D / kNT;   // D is a multiple of 256 (64 x heads, heads % 4 == 0 checked at launch)
    float qv[kRowQPerThread];
#pragma unroll
    for (int j = 0; j < kRowQPerThread; j++) qv[j] = src[min(tid + kNT * j, D - 1)];
    const float qh = src[h0 * kHeadDim + d];
    const float kx = src[D + g * kHeadDim + d];
    const float vx = src[D + KVD + g * kHeadDim + d];
    const float sk = p.kv_sk[p.layer * p.n_kv + g], sv = p.kv_sv[p.layer * p.n_kv + g];
    // ... then the cached K/V rows of this wavefront's first KPF blocks (rows
    //    0..pos-1 are final; block indices clamped inside the plane, surplus
    //    copies unused)
    v4i kreg[KPF][4], vreg[KPF][4];
#pragma unroll
    for (int i = 0; i < KPF; i++) {
        const int b = min(wave + NW * i, nblk - 1);
#pragma unroll
        for (int q = 0; q < 4; q++) kreg[i][q] = ld16(kp + (int64_t)b * 4096 + q * 1024 + lane * 16);
#pragma unroll
        for (int q = 0; q < 4; q++) vreg[i][q] = ld16(vp + (int64_t)(4 * b + q) * 1024 + lane * 16);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2) RoPE of every Q element -> row maximum
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < kRowQPerThread; j++) {
        const float o = lane_xor<32>(qv[j]);
        const float rot = d < 32 ? -o : o;
        if (j < nq) mx = fmaxf(mx, fabsf((qv[j] * cs) + (rot * sn)));
    }
    mx = wave_max_f32(mx);
    if (lane == 0) red[wave] = mx;
    // this head's rotated Q, this row's K (RoPE, static scale) and V
    const float qo = lane_xor<32>(qh), ko = lane_xor<32>(kx);
    const float qr = (qh * cs) + ((d < 32 ? -qo : qo) * sn);
    const float kr = (kx * cs) + ((d < 32 ? -ko : ko) * sn);
    const int8_t k8 = sat_i8(__builtin_rintf(__fdiv_rn(kr, sk)));
    const int8_t v8 = sat_i8(__builtin_rintf(__fdiv_rn(vx, sv)));
    kn[wave][d] = k8;
    if (h0 % G == 0 && wave == 0) {   // the first query head of the KV head appends the row
        p.kv.k[pl + KvGeom::k_off(pos, d)] = k8;
        p.kv.v[pl + KvGeom::v_off(pos, d)] = v8;
    }
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const double s_q = quant_scale(mx);
    qs[wave][d] = sat_i8(__builtin_rintf(__fdiv_rn(qr, (float)s_q)));
    const float scl = (float)((s_q * (double)sk) * p.attn_scale);
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");   // qs, kn: written and read by this wavefront

    // 3) scores of this wavefront's keys (lane <-> key); the head's INT8 Q
    //    is read from LDS once (the score stores below could alias it)
    const v4i* q4 = (const v4i*)qs[wave];
    const v4i* kn4 = (const v4i*)kn[wave];
    const v4i qa = q4[0], qb = q4[1], qc = q4[2], qd = q4[3];
    float lmax = -INFINITY;
    // key t = 64 b + lane's score, then exponential, lives in out: a register
    // for the KPF prefetched blocks of this wavefront, s_buf past them
    float se[KPF];
    auto score_block = [&](int b, v4i k0, v4i k1, v4i k2, v4i k3, float& out) {
        const int t = b * 64 + lane;
        if (t < T) {
            if (t == pos) {
                k0 = kn4[0];
                k1 = kn4[1];
                k2 = kn4[2];
                k3 = kn4[3];
            }
            int S = sdot4v(k0, qa, 0);
            S = sdot4v(k1, qb, S);
            S = sdot4v(k2, qc, S);
            S = sdot4v(k3, qd, S);
            const float s = (float)S * scl;
            out = s;
            lmax = fmaxf(lmax, s);
        }
    };
#pragma unroll
    for (int i = 0; i < KPF; i++)
        if (wave + NW * i < nblk) score_block(wave + NW * i, kreg[i][0], kreg[i][1], kreg[i][2], kreg[i][3], se[i]);
    for (int b0 = wave + NW * KPF; b0 < nblk; b0 += NW * KB) {
        v4i kk[KB][4];
#pragma unroll
        for (int i = 0; i < KB; i++) {
            const int8_t* kb = kp + (int64_t)min(b0 + NW * i, nblk - 1) * 4096 + lane * 16;
#pragma unroll
            for (int q = 0; q < 4; q++) kk[i][q] = ld16(kb + q * 1024);
        }
#pragma unroll
        for (int i = 0; i < KB; i++)
            if (b0 + NW * i < nblk)
                score_block(b0 + NW * i, kk[i][0], kk[i][1], kk[i][2], kk[i][3], s_buf[(b0 + NW * i) * 64 + lane]);
    }
    lmax = wave_max_f32(lmax);
    if (lane == 0) wmax[wave] = lmax;
    __syncthreads();
    const float m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));

    // 4) exponentials and block-64 butterfly sums of this wavefront's keys
    auto exp_block = [&](int b, float& x) {
        const int t = b * 64 + lane;
        float e = 0.0f;
        if (t < T) {   // x - max <= 0: tl_expf_nonpos is tl_expf there
            e = tl_expf_nonpos(x - m);
            x = e;
        }
        const float bs = wave_butterfly_sum(e);
        if (lane == 0) bsum[b] = bs;
    };
#pragma unroll
    for (int i = 0; i < KPF; i++)
        if (wave + NW * i < nblk) exp_block(wave + NW * i, se[i]);
    for (int b = wave + NW * KPF; b < nblk; b += NW) exp_block(b, s_buf[b * 64 + lane]);
    __syncthreads();
    const float tot = ordered_sum_aligned(bsum, nblk);   // bsum: 16-byte aligned, 16 bytes of slack

    // 5) INT8 probabilities of this wavefront's keys (exponential / total,
    //    correctly rounded: e <= 1 <= total keeps e y finite; e <= total, so
    //    rne(127 e / total) lies in [0, 127] with no clamp), then P . V over
    //    the same keys (lane <-> dimension; this row's V is v8 of lane d)
    const RnDiv dt = rn_div_prep(tot);
    auto probs = [&](auto fast) {
        auto prob_block = [&](int b, const float& x) {
            const int t = b * 64 + lane;
            int8_t pq = 0;
            if (t < T) {
                const float q = decltype(fast)::value ? rn_div_fast(x, dt) : __fdiv_rn(x, tot);
                pq = (int8_t)(int)__builtin_rintf(q * 127.0f);
            }
            p8[t] = pq;
        };
#pragma unroll
        for (int i = 0; i < KPF; i++)
            if (wave + NW * i < nblk) prob_block(wave + NW * i, se[i]);
        for (int b = wave + NW * KPF; b < nblk; b += NW) prob_block(b, s_buf[b * 64 + lane]);
    };
    if (dt.fast) probs(std::true_type{});
    else probs(std::false_type{});
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");   // p8 of these keys: this wavefront's
    int o = 0;
    const int cpos = pos >> 4, bpos = pos & 15;
    auto pv_group = [&](int c, v4i vv) {
        if (c == cpos) {
            const unsigned nb = (uint8_t)v8;
            const int sh = (bpos & 3) * 8;
            const unsigned keep = ~(0xFFu << sh);
            const int q = bpos >> 2;
            vv[q] = (int)(((unsigned)vv[q] & keep) | (nb << sh));
        }
        o = sdot4v(vv, *(const v4i*)(p8 + c * 16), o);
    };
#pragma unroll
    for (int i = 0; i < KPF; i++) {
        const int b = wave + NW * i;
        if (b < nblk)
#pragma unroll
            for (int q = 0; q < 4; q++) pv_group(4 * b + q, vreg[i][q]);
    }
    for (int b0 = wave + NW * KPF; b0 < nblk; b0 += NW * KB) {
        v4i vv[KB][4];
#pragma unroll
        for (int i = 0; i < KB; i++) {
            const int b = min(b0 + NW * i, nblk - 1);
#pragma unroll
            for (int q = 0; q < 4; q++) vv[i][q] = ld16(vp + (int64_t)(4 * b + q) * 1024 + lane * 16);
        }
#pragma unroll
        for (int i = 0; i < KB; i++)
            if (b0 + NW * i < nblk)
#pragma unroll
                for (int q = 0; q < 4; q++) pv_group(4 * (b0 + NW * i) + q, vv[i][q]);
    }
    accs[wave][lane] = o;
    __syncthreads();
    if (tid < 64) {
        const int O = accs[0][tid] + accs[1][tid] + accs[2][tid] + accs[3][tid];
        p.out[(int64_t)row * D + (int64_t)h0 * kHeadDim + tid] = (float)O * deq_mult(1.0 / 127.0, sv);
    }
}

// Batched decode attention (many rows, long contexts): one workgroup of 16
// wavefronts per (row, group of HPW = 4 query heads sharing a KV head).  The
// Q.K scores and the P.V sums run on v_mfma_i32_16x16x64_i8 with the four
// heads as rows 0, 4, 8 and 12 of the 16-row A operand (the other rows zero),
// so accumulator register 0 of lane l holds head l / 16 at column l % 16: a
// wavefront keeps every (head, key) value it computes in all 64 lanes, one
// 16-lane row per head.  Wavefront w owns key blocks b = w + 16 i (64 keys,
// i < 2): per block four MFMAs of 16 keys for the scores (lane l: keys
// 16 j + l % 16, j < 4, of head l / 16) and, per 16 output dimensions, one
// MFMA over the block's 64 keys for P.V.  Every wavefront issues all of its
// key and value loads first (T <= 2048), so each phase costs about one
// memory latency.  Same arithmetic as attention_row_kernel: the integer dot
// products are exact in any order, and the block sums keep the block-64
// butterfly order (levels 32 and 16 inside a lane's registers, 8, 4, 2, 1
// across its row).
constexpr int kGW = 16;                         // wavefronts
constexpr int kGKB = 2;                         // key blocks of 64 per wavefront
constexpr int kGroupMaxKeys = kGW * kGKB * 64;  // 2048

template <int HPW>
__global__ __launch_bounds__(kGW * 64) void attention_group_kernel(AttnDecodeArgs p) {
    static_assert(HPW == 4, "one head per 16-lane row of the MFMA accumulators");
    extern __shared__ __align__(16) float gdyn[];
    __shared__ __align__(16) int8_t qs[HPW][64];
    __shared__ __align__(16) int8_t kn[64];
    __shared__ __align__(16) int8_t vn[64];
    __shared__ float red[kGW];
    __shared__ float wmax[kGW][HPW];
    __shared__ float mh[HPW], toth[HPW];

    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int hl = lane >> 4, cl = lane & 15;   // the lane's head (row of 16 lanes) and column
    const int G = p.n_heads / p.n_kv;
    // workgroups are dispatched to the 8 XCDs round-robin by linear id: the
    // G / HPW workgroups of one (row, KV head), which read the same K and V
    // planes, get linear ids 8 apart so that they run on one XCD and share its
    // L2 (identity order when the grid is not a multiple of 8)
    int h0 = blockIdx.x * HPW, row = blockIdx.y;
    {
        const int total = gridDim.x * gridDim.y, lin = blockIdx.x + gridDim.x * blockIdx.y;
        if (total % 8 == 0) {
            const int q = (lin % 8) * (total / 8) + lin / 8, per = G / HPW;
            const int unit = q / per;
            row = unit / p.n_kv;
            h0 = (unit % p.n_kv) * G + (q % per) * HPW;
        }
    }
    const int g = h0 / G;
    const int D = p.n_heads * kHeadDim, KVD = p.n_kv * kHeadDim, W = D + 2 * KVD;
    const int pos = p.rm.pos[row], seq = p.rm.seq[row];
    if (pos < 0 || pos >= p.kv.max_pos) return;   // a row outside the cache (uniform per workgroup)
    const int T = pos + 1, tpad = (T + 63) & ~63, nblk = tpad >> 6;
    const int64_t pl = p.kv.plane(seq, p.layer, g);
    const int8_t* kp = p.kv.k + pl;
    const int8_t* vp = p.kv.v + pl;
    int8_t* p8 = (int8_t*)gdyn;                           // [HPW][tpad]
    float* bsum = (float*)(p8 + HPW * tpad);              // [HPW][nblk]
    int* accs = (int*)(bsum + HPW * nblk);                // [kGW][HPW][64]
    const bool sums = p.qacc != nullptr;   // uniform
    const double qsx = sums ? p.qas[row] : 0.0;
    // one load path for both forms, so that no load waits on another: the
    // row's 32-bit words (integer sums, or the float values' bits) and, for
    // sums, the column multipliers (for floats a second copy of the row,
    // unused)
    const int32_t* srcw = sums ? p.qacc + (int64_t)row * W : (const int32_t*)(p.qkv + (int64_t)row * W);
    const float* srcm = sums ? p.qws : p.qkv + (int64_t)row * W;
    auto qkv_val = [&](int32_t wv, float m) -> float {
        return sums ? (float)wv * deq_mult(qsx, m) : __int_as_float(wv);
    };
    const int d = lane;

    // 0) loads in the order they are needed (loads complete in issue order),
    //    all issued before any is used: the Q row, this group's Q heads and the
    //    row's own K and V (every wavefront loads them, unconditionally), the
    //    RoPE factors, then this wavefront's key operands (blocks clamped
    //    inside the plane; rows 0..pos-1 are final, surplus copies unused):
    //    key operand j of block b: keys 64 b + 16 j + l % 16, dimensions
    //    16 (l / 16) .. +16 (K plane: dimension group l / 16 of the block).
    //    A wavefront's 16 KB of key and value loads stall its instruction
    //    issue while the CU drains them, so the value operands (dimension
    //    16 j + l % 16 of keys 64 b + 16 (l / 16) .. +16, V plane group
    //    4 b + l / 16) are requested later, one block before the scores and
    //    one before the probabilities, where their issue delays less:
    //    measured per workgroup at 2048 keys, 13.4 us with every load at the
    //    start, 11.9 with all value loads before the scores, 11.4 split
    constexpr int kQPer = 4;   // Q elements per thread: D <= 4 x 1024
    int32_t qw[kQPer + 3];
    float qm[kQPer + 3];
#pragma unroll
    for (int j = 0; j < kQPer; j++) {
        const int i = min(tid + kGW * 64 * j, D - 1);
        qw[j] = srcw[i];
        qm[j] = srcm[i];
    }
    {
        const int iq = (h0 + min(wave, HPW - 1)) * kHeadDim + d, ik = D + g * kHeadDim + d, iv = ik + KVD;
        qw[kQPer] = srcw[iq];
        qm[kQPer] = srcm[iq];
        qw[kQPer + 1] = srcw[ik];
        qm[kQPer + 1] = srcm[ik];
        qw[kQPer + 2] = srcw[iv];
        qm[kQPer + 2] = srcm[iv];
    }
    const float cs = p.cosb[(int64_t)pos * kHeadDim + d];
    const float sn = p.sinb[(int64_t)pos * kHeadDim + d];
    v4i kreg[kGKB][4], vreg[kGKB][4];
#pragma unroll
    for (int i = 0; i < kGKB; i++) {
        const int b = min(wave + kGW * i, nblk - 1);
#pragma unroll
        for (int j = 0; j < 4; j++) kreg[i][j] = ld16(kp + (int64_t)b * 4096 + hl * 1024 + (16 * j + cl) * 16);
    }
    auto v_load = [&](int i) {
        const int b = min(wave + kGW * i, nblk - 1);
#pragma unroll
        for (int j = 0; j < 4; j++) vreg[i][j] = ld16(vp + (int64_t)(4 * b + hl) * 1024 + (16 * j + cl) * 16);
    };
    __builtin_amdgcn_sched_barrier(0);
    float qv[kQPer];
#pragma unroll
    for (int j = 0; j < kQPer; j++) qv[j] = qkv_val(qw[j], qm[j]);
    const float qh = qkv_val(qw[kQPer], qm[kQPer]);
    const float kx = qkv_val(qw[kQPer + 1], qm[kQPer + 1]);
    const float vx = qkv_val(qw[kQPer + 2], qm[kQPer + 2]);

    // 1) RoPE of every Q element of the row -> the row's scale; this group's
    //    rotated Q and the row's K (RoPE, static scale) and V
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < kQPer; j++) {
        const float o = lane_xor<32>(qv[j]);
        if (tid + kGW * 64 * j < D) mx = fmaxf(mx, fabsf((qv[j] * cs) + ((d < 32 ? -o : o) * sn)));
    }
    mx = wave_max_f32(mx);
    if (lane == 0) red[wave] = mx;
    const float sk = p.kv_sk[p.layer * p.n_kv + g], sv = p.kv_sv[p.layer * p.n_kv + g];
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < kGW; w++) mx = fmaxf(mx, red[w]);
    const double s_q = quant_scale(mx);
    if (wave < HPW) {
        const float qo = lane_xor<32>(qh);
        const float qr = (qh * cs) + ((d < 32 ? -qo : qo) * sn);
        qs[wave][d] = sat_i8(__builtin_rintf(__fdiv_rn(qr, (float)s_q)));
    } else if (wave == HPW) {
        const float ko = lane_xor<32>(kx);
        const float kr = (kx * cs) + ((d < 32 ? -ko : ko) * sn);
        const int8_t k8 = sat_i8(__builtin_rintf(__fdiv_rn(kr, sk)));
        const int8_t v8 = sat_i8(__builtin_rintf(__fdiv_rn(vx, sv)));
        kn[d] = k8;
        vn[d] = v8;
        if (h0 % G == 0) {   // the first head group of the KV head appends the row
            p.kv.k[pl + KvGeom::k_off(pos, d)] = k8;
            p.kv.v[pl + KvGeom::v_off(pos, d)] = v8;
        }
    }
    const float scl = (float)((s_q * (double)sk) * p.attn_scale);
    __syncthreads();

    // 2) scores: A = rotated Q (row 4 h = head h, dimensions 16 (l / 16) ..
    //    +16 from lane l), B = the key operands, the row's own key in place of
    //    the cache's at key pos
    v_load(0);
    const v4i vzero = {0, 0, 0, 0};
    const v4i qrow = *(const v4i*)&qs[cl >> 2][16 * hl];
    const v4i qa = (cl & 3) == 0 ? qrow : vzero;
    const v4i kown = *(const v4i*)&kn[16 * hl];
    float se[kGKB][4];
    float lmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < kGKB; i++) {
        const int b = wave + kGW * i;
        if (b < nblk) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int t = b * 64 + 16 * j + cl;
                const v4i kb = t == pos ? kown : kreg[i][j];
                const v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa, kb, vzero, 0, 0, 0);
                const float sc = (float)c[0] * scl;
                se[i][j] = sc;
                if (t < T) lmax = fmaxf(lmax, sc);
            }
        }
    }
    // the head's maximum over the row's 16 lanes
    lmax = fmaxf(lmax, __int_as_float(dpp<kDppXor1>(__float_as_int(lmax))));
    lmax = fmaxf(lmax, __int_as_float(dpp<kDppXor2>(__float_as_int(lmax))));
    lmax = fmaxf(lmax, __int_as_float(dpp<kDppHalfMirror>(__float_as_int(lmax))));
    lmax = fmaxf(lmax, __int_as_float(dpp<kDppRowMirror>(__float_as_int(lmax))));
    if (cl == 0) wmax[wave][hl] = lmax;
    __syncthreads();
    if (tid < HPW) {
        float m = wmax[0][tid];
        for (int w = 1; w < kGW; w++) m = fmaxf(m, wmax[w][tid]);
        mh[tid] = m;
    }
    __syncthreads();

    // 3) exponentials and block-64 butterfly sums: key 16 j + c of a block
    //    meets 16 (j ^ 2) + c (level 32), then 16 (j ^ 1) + c (level 16) in
    //    this lane's registers, then lanes c ^ 8, 4, 2, 1 of its row
    const float mhh = mh[hl];
#pragma unroll
    for (int i = 0; i < kGKB; i++) {
        const int b = wave + kGW * i;
        if (b < nblk) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int t = b * 64 + 16 * j + cl;
                // x - max <= 0: tl_expf_nonpos is tl_expf there
                se[i][j] = t < T ? tl_expf_nonpos(se[i][j] - mhh) : 0.0f;
            }
            float s = (se[i][0] + se[i][2]) + (se[i][1] + se[i][3]);
            s = s + lane_xor<8>(s);
            s = s + lane_xor<4>(s);
            s = s + lane_xor<2>(s);
            s = s + lane_xor<1>(s);
            if (cl == 0) bsum[hl * nblk + b] = s;
        }
    }
    __syncthreads();
    if (tid < HPW) {
        toth[tid] = ordered_sum(bsum + tid * nblk, nblk);
    }
    __syncthreads();

    // 4) INT8 probabilities (zero past the last key): exponential / total
    //    correctly rounded from the head's reciprocal and two residual
    //    corrections (e <= 1 <= total keeps e y finite).  A float sum of
    //    nonnegative terms is never below any of them, so e <= total and
    //    rne(127 e / total) lies in [0, 127]: the probability clip needs no
    //    clamp.
    v_load(1);
    bool fast = true;
#pragma unroll
    for (int h = 0; h < HPW; h++) fast = fast && rn_div_prep(toth[h]).fast;
    RnDiv dt;
    dt.b = toth[hl];
    dt.y = __fdiv_rn(1.0f, dt.b);
    dt.fast = fast;
    auto probs = [&](auto fst) {
#pragma unroll
        for (int i = 0; i < kGKB; i++) {
            const int b = wave + kGW * i;
            if (b < nblk) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int t = b * 64 + 16 * j + cl;
                    const float e = se[i][j];
                    const float q = decltype(fst)::value ? rn_div_fast(e, dt) : __fdiv_rn(e, dt.b);
                    p8[hl * tpad + t] = t < T ? (int8_t)(int)__builtin_rintf(q * 127.0f) : (int8_t)0;
                }
            }
        }
    };
    if (fast) probs(std::true_type{});
    else probs(std::false_type{});
    __syncthreads();

    // 5) P . V: A = the probabilities (row 4 h = head h, keys 64 b + 16 (l / 16)
    //    .. +16 from lane l), B = the value operands, the row's own V byte in
    //    place of the cache's at key pos; accumulator j, register 0 of lane l:
    //    head l / 16, dimension 16 j + l % 16
    v4i oacc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) oacc[j] = vzero;
    const int gpos = pos >> 4, bq = (pos & 15) >> 2, bsh = (pos & 3) * 8;
#pragma unroll
    for (int i = 0; i < kGKB; i++) {
        const int b = wave + kGW * i;
        if (b < nblk) {
            const v4i prow = *(const v4i*)(p8 + (cl >> 2) * tpad + b * 64 + 16 * hl);
            const v4i pa = (cl & 3) == 0 ? prow : vzero;
            const bool own = 4 * b + hl == gpos;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v4i vv = vreg[i][j];
                const unsigned nb = (uint8_t)vn[16 * j + cl];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const unsigned rep = ((unsigned)vv[q] & ~(0xFFu << bsh)) | (nb << bsh);
                    vv[q] = own && q == bq ? (int)rep : vv[q];
                }
                oacc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(pa, vv, oacc[j], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) accs[(wave * HPW + hl) * 64 + 16 * j + cl] = oacc[j][0];
    __syncthreads();
    if (tid < HPW * 64) {   // wavefront h: head h0 + h
        const int h = tid >> 6, dd = tid & 63;
        int O = 0;
        for (int w = 0; w < kGW; w++) O += accs[(w * HPW + h) * 64 + dd];
        const float v = (float)O * deq_mult(1.0 / 127.0, sv);
        p.out[(int64_t)row * D + (int64_t)(h0 + h) * kHeadDim + dd] = v;
        if (p.out_max) {   // the head's part of the maximum the O projection quantizes the row at
            const float m = wave_max_f32(fabsf(v));
            if (dd == 0) p.out_max[(int64_t)row * p.n_heads + h0 + h] = m;
        }
    }
}

static size_t group_lds_bytes(int hpw, int tpad) {
    return (size_t)hpw * tpad + (size_t)hpw * (tpad / 64) * 4 + (size_t)kGW * hpw * 64 * 4 + 16;
}

// embedding of each row's current token and the row's position (= its
// sequence's cursor) for this step
__global__ __launch_bounds__(256) void embed_step_kernel(const int32_t* __restrict__ tok_by_seq,
                                                         const int32_t* __restrict__ seq_of_row,
                                                         const int32_t* __restrict__ cursor,
                                                         int32_t* __restrict__ row_pos, int32_t d, int32_t vocab,
                                                         const int8_t* __restrict__ emb,
                                                         const float* __restrict__ emb_s, float* __restrict__ x) {
    const int row = blockIdx.x;
    const int seq = seq_of_row[row];
    const int tok = tok_by_seq[seq];
    if (threadIdx.x == 0) row_pos[row] = cursor[seq];
    if (tok < 0 || tok >= vocab) {
        for (int i = threadIdx.x; i < d; i += blockDim.x) x[(int64_t)row * d + i] = 0.0f;
        return;
    }
    const int8_t* e = emb + (int64_t)tok * d;
    const float s = emb_s[tok];
    for (int i = threadIdx.x; i < d; i += blockDim.x) x[(int64_t)row * d + i] = (float)e[i] * s;
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
static inline int cdiv(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

static int gemv_fused_rows(int pro, int epi, int kch);

template <int PRO, int EPI, int R>
static hipError_t gemv_fused_r(hipStream_t s, const GemvArgs& a) {
    const int kch = cdiv(a.k, 1024);
    const dim3 grid(cdiv(a.n, kNW * R)), block(kNT);
    // the caller sized wg_keys by gemv_fused_workgroups
    if (a.wg_keys && (int)grid.x != gemv_fused_workgroups(PRO, EPI, a.n, a.k)) return hipErrorInvalidValue;
    switch (kch) {
        case 1: TL_KLAUNCH((gemv_fused_kernel<PRO, EPI, R, 1>), grid, block, 0, s, a); break;
        case 2: TL_KLAUNCH((gemv_fused_kernel<PRO, EPI, R, 2>), grid, block, 0, s, a); break;
        case 3: TL_KLAUNCH((gemv_fused_kernel<PRO, EPI, R, 3>), grid, block, 0, s, a); break;
        case 4: TL_KLAUNCH((gemv_fused_kernel<PRO, EPI, R, 4>), grid, block, 0, s, a); break;
        case 5: TL_KLAUNCH((gemv_fused_kernel<PRO, EPI, R, 5>), grid, block, 0, s, a); break;
        case 6: TL_KLAUNCH((gemv_fused_kernel<PRO, EPI, R, 6>), grid, block, 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

static int gemv_fused_rows(int pro, int epi, int kch) {
    if (pro == PRO_RMSNORM) {
        if (epi == EPI_DEQUANT || epi == EPI_GLU) return kch <= 2 ? 3 : 1;
        if (epi == EPI_ARGMAX) return kch <= 2 ? 12 : 2;
    } else if (pro == PRO_QUANT) {
        if (epi == EPI_DEQUANT_RES) return 2;
        if (epi == EPI_DEQUANT) return kch <= 2 ? 2 : 1;
    }
    return 0;
}

int32_t gemv_fused_workgroups(int pro, int epi, int32_t n, int32_t k) {
    const int r = gemv_fused_rows(pro, epi, cdiv(k, 1024));
    return r > 0 ? cdiv(n, kNW * r) : 0;
}

int64_t gemv_fused_wavefronts(int pro, int epi, int32_t n, int32_t k) {
    return (int64_t)gemv_fused_workgroups(pro, epi, n, k) * kNW;
}

hipError_t launch_gemv_fused(hipStream_t s, int pro, int epi, const GemvArgs& a) {
    if (a.n <= 0) return hipSuccess;
    if (a.k <= 0 || a.k % 64 != 0 || a.k > 6 * 1024) return hipErrorInvalidValue;
    if (pro == PRO_RMSNORM && (a.plan.n_leaves > 64 || a.plan.leaf_len * a.plan.n_leaves != a.k)) return hipErrorInvalidValue;
    const int kch = cdiv(a.k, 1024);
#define TL_GO(P, E, R) return gemv_fused_r<P, E, R>(s, a)
    // rows per wavefront measured fastest (graph replay over rotating weights) for the
    // TinyLlama shapes: Q|K|V 3, gate/up 3, LM head 12, O 2, down 2
    if (pro == PRO_RMSNORM) {
        if (epi == EPI_DEQUANT) { if (kch <= 2) TL_GO(PRO_RMSNORM, EPI_DEQUANT, 3); TL_GO(PRO_RMSNORM, EPI_DEQUANT, 1); }
        if (epi == EPI_GLU) { if (kch <= 2) TL_GO(PRO_RMSNORM, EPI_GLU, 3); TL_GO(PRO_RMSNORM, EPI_GLU, 1); }
        if (epi == EPI_ARGMAX) { if (kch <= 2) TL_GO(PRO_RMSNORM, EPI_ARGMAX, 12); TL_GO(PRO_RMSNORM, EPI_ARGMAX, 2); }
    } else if (pro == PRO_QUANT) {
        if (epi == EPI_DEQUANT_RES) TL_GO(PRO_QUANT, EPI_DEQUANT_RES, 2);
        if (epi == EPI_DEQUANT) { if (kch <= 2) TL_GO(PRO_QUANT, EPI_DEQUANT, 2); TL_GO(PRO_QUANT, EPI_DEQUANT, 1); }
    }
#undef TL_GO
    return hipErrorInvalidValue;
}

bool attention_decode_grouped(int32_t rows, int32_t n_heads, int32_t n_kv, int32_t max_t) {
    if (rows <= 1 || n_kv <= 0 || n_heads % n_kv || n_heads > 32 * 4) return false;
    const int G = n_heads / n_kv, D = n_heads * kHeadDim;
    return G <= kMaxGroupHeads && G % 4 == 0 && max_t <= kGroupMaxKeys && D <= 4 * kGW * 64;
}

hipError_t launch_attention_decode(hipStream_t s, const float* qkv, int32_t rows, int32_t n_heads, int32_t n_kv,
                                   RowMap rm, const float* cos, const float* sin, KvGeom kv, int32_t layer,
                                   const float* kv_sk, const float* kv_sv, float* out, int32_t max_t,
                                   unsigned long long* ts, const QkvSums* sums, float* out_max) {
    if (rows <= 0) return hipSuccess;
    const int G = n_heads / n_kv;
    if (n_heads % n_kv || G > kMaxGroupHeads || n_heads > 32 * 4) return hipErrorInvalidValue;
    const int D = n_heads * kHeadDim, W = D + 2 * n_kv * kHeadDim;
    const int tpad = (max_t + 63) & ~63;
    AttnDecodeArgs p{qkv, n_heads, n_kv, rm, cos, sin, kv, layer, kv_sk, kv_sv, 1.0 / sqrt((double)kHeadDim), out, ts,
                     nullptr, nullptr, nullptr, nullptr};
    const bool grouped = attention_decode_grouped(rows, n_heads, n_kv, max_t);
    if (out_max && !grouped) return hipErrorInvalidValue;
    p.out_max = out_max;
    if (sums) {
        if (!grouped || !sums->acc || !sums->as || !sums->ws) return hipErrorInvalidValue;
        p.qacc = sums->acc;
        p.qas = sums->as;
        p.qws = sums->ws;
    }
    if (grouped) {
        // many rows: the grouped kernel, 4 query heads per workgroup (with 8
        // per workgroup, one per KV head, it measured slower: half the
        // workgroups, longer phases)
        TL_KLAUNCH((attention_group_kernel<4>), dim3(n_heads / 4, rows), dim3(kGW * 64), group_lds_bytes(4, tpad), s,
                   p);
    } else if (n_heads % 4 == 0 && D <= kRowQPerThread * kNT) {
        const size_t lds = (size_t)tpad * 5 + (tpad / 64) * 4 + 16;
        TL_KLAUNCH((attention_row_kernel<2>), dim3(n_heads, rows), dim3(256), lds, s, p);
    } else {
        const size_t lds = sizeof(float) * W + (size_t)tpad * 4 + tpad + (tpad / 64) * 4 + 64;
        TL_KLAUNCH((attention_decode_kernel<1, 2, 8, 4>), dim3(n_heads, rows), dim3(256), lds, s, p);
    }
    return hipGetLastError();
}

hipError_t launch_embed_step(hipStream_t s, const int32_t* tok_by_seq, const int32_t* seq_of_row, int32_t rows,
                             const int32_t* cursor, int32_t* row_pos, int32_t d, int32_t vocab, const int8_t* emb,
                             const float* emb_s, float* x) {
    if (rows <= 0) return hipSuccess;
    TL_KLAUNCH(embed_step_kernel, dim3(rows), dim3(256), 0, s, tok_by_seq, seq_of_row, cursor, row_pos, d,
                       vocab, emb, emb_s, x);
    return hipGetLastError();
}

hipError_t init_decode_kernels() {
    hipError_t e = hipFuncSetAttribute((const void*)attention_row_kernel<2>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 120 * 1024);
    if (e != hipSuccess) return e;
    e = hipFuncSetAttribute((const void*)attention_group_kernel<4>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)group_lds_bytes(4, kGroupMaxKeys));
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute((const void*)attention_decode_kernel<1, 2, 8, 4>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024);
}

}  // namespace tl
