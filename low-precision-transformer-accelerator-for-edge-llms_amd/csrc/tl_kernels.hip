// tl_kernels.hip -- hand-written HIP kernels for gfx950 (MI355X) implementing
// the shared INT8 TinyLlama decoder path of the reference
// (model/tinyllama_gemm_int8.py, rtl/compute/*.sv).
//
// Numerical contract (identical, operation by operation, to oracle/tl_oracle.c):
//   * INT8 x INT8 -> INT32 contractions are exact (v_dot4 / v_mfma_i32_*_i8);
//   * float32 arithmetic is never contracted into FMAs (built with
//     -ffp-contract=off); divisions and square roots are correctly rounded;
//   * every float reduction uses a fixed order: NumPy's pairwise tree for the
//     RMSNorm sum of squares, a 64-wide xor butterfly per block of 64 keys
//     followed by an in-order sum over blocks for the softmax denominator;
//   * maxima, integer sums and the argmax key are order independent.
// With these, results are bit-identical to the oracle.

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>

#include "tl_device.h"
#include "tl_internal.h"
#include "tl_prologue.h"

namespace tl {

// ---------------------------------------------------------------------------
// RMSNorm + per-row INT8 quantization (TL:45-50, GI:36-42)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rmsnorm_quant_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ g, int32_t n,
                                                            float eps, PwPlan plan,
                                                            float* __restrict__ y,
                                                            int8_t* __restrict__ q,
                                                            double* __restrict__ scales) {
    extern __shared__ float lds[];
    float* xs = lds;
    float* sq = lds + n;
    float* scr = sq + n;
    const int row = blockIdx.x, tid = threadIdx.x;
    const float* xr = x + (int64_t)row * n;
    for (int i = tid; i < n; i += blockDim.x) {
        float v = xr[i];
        xs[i] = v;
        sq[i] = v * v;
    }
    __syncthreads();
    const float sum = block_pairwise_sum(sq, plan, scr);
    const float var = __fdiv_rn(sum, (float)n);
    const float inv = __fdiv_rn(1.0f, __builtin_sqrtf(var + eps));
    float mx = 0.0f;
    for (int i = tid; i < n; i += blockDim.x) {
        float a = (xs[i] * inv) * g[i];
        xs[i] = a;
        mx = fmaxf(mx, fabsf(a));
        if (y) y[(int64_t)row * n + i] = a;
    }
    mx = block_max(mx, scr);
    const double s = quant_scale(mx);
    const float sf = (float)s;
    for (int i = tid; i < n; i += blockDim.x) q[(int64_t)row * n + i] = sat_i8(__builtin_rintf(__fdiv_rn(xs[i], sf)));
    if (tid == 0) scales[row] = s;
}

// per-row quantize_int8 (GI:36-42); float scales variant is the offline
// per-output-channel weight quantizer
template <bool FLOAT_SCALE>
__global__ __launch_bounds__(256) void quantize_rows_kernel(const float* __restrict__ x, int32_t n,
                                                            int8_t* __restrict__ q, void* scales) {
    __shared__ float red[16];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float* xr = x + (int64_t)row * n;
    float mx = 0.0f;
    for (int i = tid; i < n; i += blockDim.x) mx = fmaxf(mx, fabsf(xr[i]));
    mx = block_max(mx, red);
    const double s = quant_scale(mx);
    const float sf = (float)s;
    for (int i = tid; i < n; i += blockDim.x) q[(int64_t)row * n + i] = sat_i8(__builtin_rintf(__fdiv_rn(xr[i], sf)));
    if (tid == 0) {
        if (FLOAT_SCALE) ((float*)scales)[row] = sf;
        else ((double*)scales)[row] = s;
    }
}

// the same two row operations for rows of width n <= 1024 KCH, n % 64 == 0,
// 16-byte aligned, one workgroup per row: float4 loads, the decode GEMV
// prologues (identical arithmetic: NumPy pairwise tree, per-row scale), and
// 16-byte stores of the INT8 row (row-major, or with pk in the packed GEMM
// operand layout: piece p of row r at ((r / 32) (n / 32) + p / 2) 1024 +
// ((p % 2) 32 + r % 32) 16).  With `zero`, the workgroup also clears zero_n
// int32 of its row of that buffer (integer sums that the kernels before it
// have consumed, zero again for the next K-sliced GEMM).
// the weight tiles of XCD xcd, split in 64 KB units over the nslots
// prefetching workgroups of that XCD (slot = this one's index): plain loads,
// a whole unit (sixteen 16-byte loads per thread) in flight at once, so the
// lines are kept in L2
TL_DEV void l2_prefetch(const L2Prefetch& pf, int xcd, int slot, int nslots) {
    constexpr int kU = 16;
    constexpr int64_t kUnit = 65536;
    const int nch = (int)((pf.tile_bytes + kUnit - 1) / kUnit);
    const int units = (pf.ntiles >> 3) * pf.nmat * nch;
    v4i acc = {0, 0, 0, 0};
    for (int u = slot; u < units; u += nslots) {
        const int c = u % nch, mt = u / nch, m = mt % pf.nmat, i = mt / pf.nmat;
        const int64_t off = (int64_t)c * kUnit;
        const int nv = (int)(min(kUnit, pf.tile_bytes - off) >> 4);
        const v4i* src = (const v4i*)(pf.w[m] + (int64_t)(xcd + 8 * i) * pf.tile_bytes + off);
        for (int o = threadIdx.x; o < nv; o += kU * kNT) {
            v4i r[kU];
#pragma unroll
            for (int j = 0; j < kU; j++) r[j] = src[min(o + j * kNT, nv - 1)];
#pragma unroll
            for (int j = 0; j < kU; j++) acc ^= r[j];
        }
    }
    if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x5EED1E55) *pf.sink = 1;
}

// prefetching workgroups per XCD for a plan (0: none): one per 64 KB unit of
// the XCD's tiles, at most 28 (with a row kernel's 32 workgroups, 256 in all)
static int l2_prefetch_slots(const L2Prefetch* pf) {
    if (!pf || !pf->w[0] || pf->ntiles <= 0 || pf->ntiles % 8 || pf->nmat < 1 || pf->nmat > 2 ||
        (pf->nmat == 2 && !pf->w[1]) || !pf->sink || pf->tile_bytes <= 0 || pf->tile_bytes % 16)
        return 0;
    const int64_t units = (int64_t)(pf->ntiles / 8) * pf->nmat * ((pf->tile_bytes + 65535) / 65536);
    return (int)std::min<int64_t>(28, units);
}

template <int PRO, int KCH>
__global__ __launch_bounds__(kNT) void rows_prologue_kernel(const float* __restrict__ x, const float* __restrict__ g,
                                                           int32_t n, float eps, PwPlan plan, int8_t* __restrict__ q,
                                                           double* __restrict__ scales, int32_t* __restrict__ zero,
                                                           int32_t zero_n, int32_t pk, int32_t rows, L2Prefetch pf) {
    __shared__ __align__(16) int8_t xs8[KCH * 1024];
    __shared__ __align__(16) float sq[PRO == PRO_RMSNORM ? KCH * 1024 : 4];
    __shared__ __align__(16) float part[PRO == PRO_RMSNORM ? 8 * 64 : 4];
    __shared__ float red[16];
    __shared__ double xscale;
    const int tid = threadIdx.x;
    // workgroups past the rows (from the next multiple of 8) prefetch
    const int rows8 = (rows + 7) & ~7;
    if ((int)blockIdx.x >= rows) {
        if ((int)blockIdx.x >= rows8)
            l2_prefetch(pf, (int)(blockIdx.x - rows8) % 8, (int)(blockIdx.x - rows8) / 8, ((int)gridDim.x - rows8) / 8);
        return;
    }
    // packed rows: workgroups go to the 8 XCDs round-robin by id, so workgroup
    // w takes row (w % 8) (rows / 8) + w / 8 and each XCD writes whole 32-row
    // blocks, whose 16-byte pieces (adjacent for consecutive rows) then meet
    // in that XCD's L2
    const int row = pk && rows % 8 == 0 ? (int)(blockIdx.x % 8) * (rows / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
    const float4* xr = (const float4*)(x + (int64_t)row * n);
    const int kq = n / 4 - 1;
    float4 xv[KCH], gv[KCH];
#pragma unroll
    for (int c = 0; c < KCH; c++) {
        const int idx = min(c * kNT + tid, kq);
        xv[c] = xr[idx];
        if (PRO == PRO_RMSNORM) gv[c] = ((const float4*)g)[idx];
    }
    if (PRO == PRO_QUANT) prologue_quant<KCH>(xv, n, xs8, red, &xscale);
    else prologue_rmsnorm<KCH>(xv, gv, n, eps, plan, sq, part, xs8, red, &xscale);
    if (pk) {
        int8_t* qt = q + (int64_t)(row >> 5) * (n >> 5) * 1024 + (row & 31) * 16;
        for (int o = tid * 16; o < n; o += kNT * 16)
            *(v4i*)(qt + (o >> 5) * 1024 + ((o >> 4) & 1) * 512) = *(const v4i*)(xs8 + o);
    } else {
        int8_t* qr = q + (int64_t)row * n;
        for (int o = tid * 16; o < n; o += kNT * 16) *(v4i*)(qr + o) = *(const v4i*)(xs8 + o);
    }
    if (tid == 0) scales[row] = xscale;
    if (zero)
        for (int i = tid * 4; i < zero_n; i += kNT * 4) *(v4i*)(zero + (int64_t)row * zero_n + i) = (v4i){0, 0, 0, 0};
}

template <int PRO>
static hipError_t launch_rows_prologue(hipStream_t s, const float* x, const float* g, int32_t rows, int32_t n,
                                       float eps, PwPlan plan, int8_t* q, double* scales, int32_t* zero = nullptr,
                                       int32_t zero_n = 0, bool packed = false, const L2Prefetch* pfp = nullptr) {
    const int slots = l2_prefetch_slots(pfp);
    const L2Prefetch pf = slots ? *pfp : L2Prefetch{};
    const dim3 grid(slots ? ((rows + 7) & ~7) + 8 * slots : rows), block(kNT);
    const int32_t pk = packed ? 1 : 0;
#define TL_RPL(C) TL_KLAUNCH((rows_prologue_kernel<PRO, C>), grid, block, 0, s, x, g, n, eps, plan, q, scales, zero, zero_n, pk, rows, pf)
    switch ((n + 1023) / 1024) {
        case 1: TL_RPL(1); break;
        case 2: TL_RPL(2); break;
        case 3: TL_RPL(3); break;
        case 4: TL_RPL(4); break;
        case 5: TL_RPL(5); break;
        case 6: TL_RPL(6); break;
        default: return hipErrorInvalidValue;
    }
#undef TL_RPL
    return hipGetLastError();
}

// the RMSNorm row prologue above, preceded by the epilogue of a K-sliced
// small-M GEMM whose workgroups added their integer sums into acc (EPI_ACC):
// gemm_rows32_kernel's DEQUANT_RES arithmetic on the complete sums, so the
// values are those of the unsliced GEMM
template <int KCH>
__global__ __launch_bounds__(kNT) void rows_fold_kernel(FoldArgs f) {
    __shared__ __align__(16) int8_t xs8[KCH * 1024];
    __shared__ __align__(16) float sq[KCH * 1024];
    __shared__ __align__(16) float part[8 * 64];
    __shared__ float red[16];
    __shared__ double xscale;
    const int tid = threadIdx.x, row = blockIdx.x, n = f.n;
    // workgroups past the rows (from the next multiple of 8) prefetch
    const int rows8 = (f.rows + 7) & ~7;
    if (row >= f.rows) {
        if (row >= rows8) l2_prefetch(f.pf, (row - rows8) % 8, (row - rows8) / 8, ((int)gridDim.x - rows8) / 8);
        return;
    }
    const int kq = n / 4 - 1;
    const int64_t ro = (int64_t)row * n;
    // f.as[row] may be the buffer this workgroup's scale is written to: every
    // thread reads it here, and uses it before the prologue's first barrier
    const double sx = f.as[row];
    v4i av[KCH];
    float4 wv[KCH], rv[KCH], gv[KCH];
#pragma unroll
    for (int c = 0; c < KCH; c++) {
        const int idx = min(c * kNT + tid, kq);
        av[c] = ((const v4i*)(f.acc + ro))[idx];
        wv[c] = ((const float4*)f.ws)[idx];
        rv[c] = ((const float4*)(f.x + ro))[idx];
        gv[c] = ((const float4*)f.g)[idx];
    }
    float4 xv[KCH];
#pragma unroll
    for (int c = 0; c < KCH; c++) {
        xv[c].x = rv[c].x + (float)av[c][0] * deq_mult(sx, wv[c].x);
        xv[c].y = rv[c].y + (float)av[c][1] * deq_mult(sx, wv[c].y);
        xv[c].z = rv[c].z + (float)av[c][2] * deq_mult(sx, wv[c].z);
        xv[c].w = rv[c].w + (float)av[c][3] * deq_mult(sx, wv[c].w);
        const int idx = c * kNT + tid;
        if (idx <= kq) {
            // each element is read and cleared by the same thread
            ((v4i*)(f.acc + ro))[idx] = (v4i){0, 0, 0, 0};
            ((float4*)(f.x + ro))[idx] = xv[c];
        }
    }
    prologue_rmsnorm<KCH>(xv, gv, n, f.eps, f.plan, sq, part, xs8, red, &xscale);
    int8_t* qr = f.q + ro;
    for (int o = tid * 16; o < n; o += kNT * 16) *(v4i*)(qr + o) = *(const v4i*)(xs8 + o);
    if (tid == 0) f.scales[row] = xscale;
    if (f.zero)
        for (int i = tid * 4; i < f.zero_n; i += kNT * 4) *(v4i*)(f.zero + (int64_t)row * f.zero_n + i) = (v4i){0, 0, 0, 0};
}

hipError_t launch_rows_fold(hipStream_t s, const FoldArgs& f) {
    if (f.rows <= 0) return hipSuccess;
    const uintptr_t bits = (uintptr_t)f.x | (uintptr_t)f.acc | (uintptr_t)f.ws | (uintptr_t)f.g | (uintptr_t)f.q;
    if (f.n <= 0 || f.n % 64 || f.n > 6 * 1024 || bits % 16 || !f.x || !f.acc || !f.as || !f.ws || !f.g || !f.q ||
        !f.scales || f.plan.n_leaves > 64)
        return hipErrorInvalidValue;
    if (f.zero && (f.zero_n <= 0 || f.zero_n % 4 || (uintptr_t)f.zero % 16)) return hipErrorInvalidValue;
    const int slots = l2_prefetch_slots(&f.pf);
    FoldArgs fa = f;
    if (!slots) fa.pf = L2Prefetch{};
    const dim3 grid(slots ? ((f.rows + 7) & ~7) + 8 * slots : f.rows), block(kNT);
    switch ((f.n + 1023) / 1024) {
        case 1: TL_KLAUNCH(rows_fold_kernel<1>, grid, block, 0, s, fa); break;
        case 2: TL_KLAUNCH(rows_fold_kernel<2>, grid, block, 0, s, fa); break;
        case 3: TL_KLAUNCH(rows_fold_kernel<3>, grid, block, 0, s, fa); break;
        case 4: TL_KLAUNCH(rows_fold_kernel<4>, grid, block, 0, s, fa); break;
        case 5: TL_KLAUNCH(rows_fold_kernel<5>, grid, block, 0, s, fa); break;
        case 6: TL_KLAUNCH(rows_fold_kernel<6>, grid, block, 0, s, fa); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

static bool rows_fast_ok(const void* x, const void* g, const void* q, int32_t n) {
    const uintptr_t bits = (uintptr_t)x | (uintptr_t)g | (uintptr_t)q;
    return n % 64 == 0 && n <= 6 * 1024 && bits % 16 == 0;
}

// per-tensor quantize_int8 over n elements (two passes: global max, then quantize)
__global__ __launch_bounds__(256) void tensor_absmax_kernel(const float* __restrict__ x, int64_t n,
                                                            unsigned* __restrict__ mx_bits) {
    __shared__ float red[16];
    float mx = 0.0f;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        mx = fmaxf(mx, fabsf(x[i]));
    mx = block_max(mx, red);
    if (threadIdx.x == 0) atomicMax(mx_bits, __float_as_uint(mx));  // |x| >= 0: bit order = value order
}

__global__ __launch_bounds__(256) void tensor_quant_kernel(const float* __restrict__ x, int64_t n,
                                                           const unsigned* __restrict__ mx_bits,
                                                           int8_t* __restrict__ q, double* __restrict__ scale) {
    const double s = quant_scale(__uint_as_float(*mx_bits));
    const float sf = (float)s;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        q[i] = sat_i8(__builtin_rintf(__fdiv_rn(x[i], sf)));
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale = s;
}

__global__ void fill_u32_kernel(unsigned* p, int32_t n, unsigned v) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// ---------------------------------------------------------------------------
// Decode GEMV (M = 1): y[n] = epilogue(sum_k x[k] * W[n][k])
// Each wavefront owns R consecutive output rows; lane l streams bytes
// [1024 c + 16 l, +16) of every row (128-bit loads, one coalesced KiB per
// wavefront instruction) and all weight loads are issued before any math.
// The dot products run on v_dot4_i32_i8 and each row sum is a wavefront
// reduction (exact integer arithmetic).
// ---------------------------------------------------------------------------
template <int R, int KCH, int EPI>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
    constexpr int NM = (EPI == EPI_GLU) ? 2 : 1;
    __shared__ unsigned long long wbest[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * 4 + wave) * R;
    const int K = a.k;

    // activation row and this lane's epilogue operands first (lane l < R
    // finishes row row0 + l), then the weight rows: unconditional 128-bit
    // loads at clamped in-bounds offsets; lanes past the end of a row meet
    // activation bytes cleared below
    v4i xv[KCH];
#pragma unroll
    for (int c = 0; c < KCH; c++) xv[c] = ld16(a.x + min(c * 1024 + lane * 16, K - 16));
    const int nl = min(row0 + min(lane, R - 1), a.n - 1);
    // (a raw-sum launch passes no multipliers)
    const float wsl = (EPI != EPI_REQUANT || a.ws) ? a.ws[nl] : 0.0f;
    const float ws2l = (EPI == EPI_GLU) ? a.ws2[nl] : 0.0f;
    const float resl = (EPI == EPI_DEQUANT_RES) ? a.residual[nl] : 0.0f;
    const double sx = (EPI == EPI_REQUANT) ? 0.0 : a.xs[0];
    __builtin_amdgcn_sched_barrier(0);
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
#pragma unroll
    for (int c = 0; c < KCH; c++)
        if (c * 1024 + lane * 16 >= K) xv[c] = (v4i){0, 0, 0, 0};
    int acc[NM][R];
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
        for (int r = 0; r < R; r++) {
            int sum = 0;
#pragma unroll
            for (int c = 0; c < KCH; c++) sum = sdot4v(wv[m][r][c], xv[c], sum);
            acc[m][r] = wave_sum_i32(sum);
        }
    // the sums are wavefront-uniform; lane l < R takes row l's
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
        if (threadIdx.x == 0) {
            unsigned long long b = wbest[0];
            for (int i = 1; i < 4; i++) b = wbest[i] > b ? wbest[i] : b;
            if (b) atomicMax(a.key, b);
        }
        return;
    }
    if (!live) return;
    if (a.acc) a.acc[n] = mine[0];
    if (EPI == EPI_REQUANT) {
        if (a.y8) a.y8[n] = sat_i8(__builtin_rintf((float)mine[0] * wsl));
    } else if (EPI == EPI_DEQUANT || EPI == EPI_DEQUANT_RES) {
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
// INT8 MFMA GEMM (M > 1): C[M][N] = A[M][K] . W[N][K]^T with
// v_mfma_i32_16x16x64_i8.  Workgroup of 4 wavefronts in a 2 x 2 grid; each
// wavefront owns a (16 WTM) x (16 WTN) output tile; K advances 64 per step
// through double-buffered LDS tiles (one 128-bit global load per thread per
// operand tile, stored with an xor swizzle so the 128-bit fragment reads are
// bank-conflict free).  Split-K writes exact int32 partials; otherwise the
// dequantization (+ residual or SiLU-GLU) epilogue is fused.
// ---------------------------------------------------------------------------
TL_DEV int swz(int row, int kc) { return row * 4 + (kc ^ ((row >> 2) & 3)); }

template <int WTM, int WTN, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs a) {
    constexpr int BM = 32 * WTM, BN = 32 * WTN;
    constexpr int NB = (EPI == EPI_GLU) ? 2 : 1;
    constexpr int ACH = BM * 4, BCH = BN * 4;   // 16-byte chunks per operand tile
    __shared__ int4 sa[2][ACH];
    __shared__ int4 sb[2][NB][BCH];

    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int kb = blockIdx.z * a.k_split;
    const int ke = min(a.k, kb + a.k_split);
    const int nsteps = (ke - kb) >> 6;

    // global -> register staging assignment
    const bool a_on = tid < ACH;
    const int a_row = tid >> 2, a_kc = tid & 3;
    const int8_t* a_src = a.a + (int64_t)min(m0 + a_row, a.m - 1) * a.k + a_kc * 16;
    const bool b_on = tid < BCH;
    const int b_row = tid >> 2, b_kc = tid & 3;
    const int8_t* b_src[NB];
#pragma unroll
    for (int b = 0; b < NB; b++)
        b_src[b] = (b ? a.w2 : a.w) + (int64_t)min(n0 + b_row, a.n - 1) * a.k + b_kc * 16;

    int4 ra = make_int4(0, 0, 0, 0), rb[NB];
    auto gload = [&](int kk) {
        if (a_on) ra = *(const int4*)(a_src + kk);
#pragma unroll
        for (int b = 0; b < NB; b++)
            if (b_on) rb[b] = *(const int4*)(b_src[b] + kk);
    };
    auto lstore = [&](int buf) {
        if (a_on) sa[buf][swz(a_row, a_kc)] = ra;
#pragma unroll
        for (int b = 0; b < NB; b++)
            if (b_on) sb[buf][b][swz(b_row, b_kc)] = rb[b];
    };

    v4i acc[NB][WTM][WTN];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int i = 0; i < WTM; i++)
#pragma unroll
            for (int j = 0; j < WTN; j++) acc[b][i][j] = (v4i){0, 0, 0, 0};

    if (nsteps > 0) {
        gload(kb);
        lstore(0);
        __syncthreads();
    }
    const int fr = lane & 15, fk = lane >> 4;
    for (int s = 0; s < nsteps; s++) {
        const int buf = s & 1;
        if (s + 1 < nsteps) gload(kb + (s + 1) * 64);
        v4i af[WTM], bf[NB][WTN];
#pragma unroll
        for (int i = 0; i < WTM; i++) {
            const int row = wm * 16 * WTM + i * 16 + fr;
            int4 t = sa[buf][swz(row, fk)];
            af[i] = (v4i){t.x, t.y, t.z, t.w};
        }
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int j = 0; j < WTN; j++) {
                const int col = wn * 16 * WTN + j * 16 + fr;
                int4 t = sb[buf][b][swz(col, fk)];
                bf[b][j] = (v4i){t.x, t.y, t.z, t.w};
            }
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int i = 0; i < WTM; i++)
#pragma unroll
                for (int j = 0; j < WTN; j++)
                    acc[b][i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[b][j], acc[b][i][j], 0, 0, 0);
        if (s + 1 < nsteps) {
            lstore(buf ^ 1);
            __syncthreads();
        }
    }

    // epilogue: lane holds C[(lane/16)*4 + e][lane%16] of each 16x16 tile
    const bool partial = gridDim.z > 1 || EPI == EPI_RAW;
#pragma unroll
    for (int i = 0; i < WTM; i++)
#pragma unroll
        for (int j = 0; j < WTN; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + wm * 16 * WTM + i * 16 + (lane >> 4) * 4 + e;
                const int n = n0 + wn * 16 * WTN + j * 16 + (lane & 15);
                if (m >= a.m || n >= a.n) continue;
                const int64_t idx = (int64_t)m * a.n + n;
                if (partial) {
                    const int64_t plane = (int64_t)a.m * a.n;
#pragma unroll
                    for (int b = 0; b < NB; b++)
                        a.acc[(int64_t)(blockIdx.z * NB + b) * plane + idx] = acc[b][i][j][e];
                    continue;
                }
                const double sx = a.as[m];
                const float v0 = (float)acc[0][i][j][e] * deq_mult(sx, a.ws[n]);
                if (EPI == EPI_GLU) {
                    const float up = (float)acc[NB - 1][i][j][e] * deq_mult(sx, a.ws2[n]);
                    a.y[idx] = tl_silu(v0) * up;
                } else if (EPI == EPI_DEQUANT_RES) {
                    a.y[idx] = a.residual[idx] + v0;
                } else {
                    a.y[idx] = v0;
                }
            }
}

// sum split-K partials (exact) and apply the epilogue
template <int EPI>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmArgs a, int32_t splits) {
    constexpr int NB = (EPI == EPI_GLU) ? 2 : 1;
    const int64_t total = (int64_t)a.m * a.n;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        int s[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            int v = 0;
            for (int z = 0; z < splits; z++) v += a.acc[(int64_t)(z * NB + b) * total + idx];
            s[b] = v;
        }
        const int m = (int)(idx / a.n), n = (int)(idx % a.n);
        if (EPI == EPI_RAW) {
            a.acc[idx] = s[0];
            continue;
        }
        const double sx = a.as[m];
        const float v0 = (float)s[0] * deq_mult(sx, a.ws[n]);
        if (EPI == EPI_GLU) {
            const float up = (float)s[NB - 1] * deq_mult(sx, a.ws2[n]);
            a.y[idx] = tl_silu(v0) * up;
        } else if (EPI == EPI_DEQUANT_RES) {
            a.y[idx] = a.residual[idx] + v0;
        } else {
            a.y[idx] = v0;
        }
    }
}

// ---------------------------------------------------------------------------
// small-M GEMM (M <= 32: batched decode rows) on i8 MFMA with the split-K
// reduction inside the kernel.  Workgroup (t, s) computes the 32 x 32 output
// tile t (all M rows, columns 32 t .. 32 t + 31) over K slice s of `slices`;
// its 4 wavefronts split the slice again and add their tiles in LDS.  With
// more than one slice the workgroup stores its partial tile (device-coherent
// stores), and the last of the tile's workgroups to arrive (per-tile counter)
// adds every partial -- exact integers, any order -- runs the epilogue of
// gemm_reduce_kernel and sets the counter back to zero for the next launch.
// A operand: lane l holds row l % 32, 16 bytes at K offset 16 (l / 32) of a
// 32-byte chunk; B operand: column (weight row) l % 32, same bytes.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(1))) void GlobalVoid;
typedef __attribute__((address_space(3))) void LdsVoid;
constexpr int kCoherentLoad = 16;   // cache policy of a device-scope coherent load (sc1)

// Operands reach LDS by device-to-LDS loads in rounds of up to 8 chunks
// (256 K bytes): one load instruction moves 4 full rows x 256 bytes, and the
// 16-byte column s of row r is stored at slot s ^ (r & 15), so the fragment
// reads (lane l: row l % 32, one 16-byte column) spread over the banks.
constexpr int kSkinnyRound = 8;   // 32-byte K chunks per round

TL_DEV void skinny_stage(const int8_t* base, int64_t stride, int rows_valid, int kbyte0, int K, int8_t* lds) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int row = 4 * i + (lane >> 4), slot = lane & 15;
        const int col = slot ^ (row & 15);
        const int8_t* src = base + (int64_t)min(row, rows_valid - 1) * stride + min(kbyte0 + col * 16, K - 16);
        __builtin_amdgcn_global_load_lds((GlobalVoid*)src, (LdsVoid*)(lds + i * 1024), 16, 0, 0);
    }
}

TL_DEV v4i skinny_frag(const int8_t* lds, int row, int col16) {
    return *(const v4i*)(lds + row * 256 + ((col16 ^ (row & 15)) << 4));
}

template <int EPI>
__global__ __launch_bounds__(256) void gemm_skinny_kernel(GemmArgs a, int32_t slices, int32_t* __restrict__ part,
                                                          unsigned* __restrict__ counters) {
    constexpr int NB = EPI == EPI_GLU ? 2 : 1;
    extern __shared__ __align__(16) int8_t skinny_lds[];   // per wavefront: A + NB weight tiles of 32 x 256 bytes
    const int tid = threadIdx.x, lane = tid & 63, col = lane & 31, hi = lane >> 5;
    const int wave = wave_id();   // uniform: LDS load bases go to a scalar register
    const int tile = blockIdx.x / slices, sl = blockIdx.x % slices;
    const int n0 = tile * 32;
    const int kch = a.k >> 5;
    const int per = (kch + slices * 4 - 1) / (slices * 4);
    const int c0 = (sl * 4 + wave) * per, c1 = min(c0 + per, kch);
    int8_t* lds_a = skinny_lds + wave * (1 + NB) * 8192;
    v16i acc[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) acc[b] = (v16i){};
    for (int c = c0; c < c1; c += kSkinnyRound) {
        const int nch = min(kSkinnyRound, c1 - c);
        skinny_stage(a.a, a.k, a.m, c * 32, a.k, lds_a);
        skinny_stage(a.w + (int64_t)n0 * a.k, a.k, a.n - n0, c * 32, a.k, lds_a + 8192);
        if (NB == 2) skinny_stage(a.w2 + (int64_t)n0 * a.k, a.k, a.n - n0, c * 32, a.k, lds_a + 16384);
        __builtin_amdgcn_s_waitcnt(0);   // this wavefront's tiles are in LDS
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
        for (int j = 0; j < kSkinnyRound; j++) {
            if (j < nch) {
                const v4i af = skinny_frag(lds_a, col, 2 * j + hi);
#pragma unroll
                for (int b = 0; b < NB; b++)
                    acc[b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, skinny_frag(lds_a + 8192 * (1 + b), col, 2 * j + hi),
                                                                   acc[b], 0, 0, 0);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");   // reads done before the next round's loads land
    }
    // wavefront partials -> LDS (the staging area is free once every wavefront is past its last round)
    __syncthreads();
    int* red = (int*)skinny_lds;   // [slices <= 8][NB][16][64]
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int i = 0; i < 16; i++) red[((wave * NB + b) * 16 + i) * 64 + lane] = acc[b][i];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int o = (b * 16 + i) * 64 + lane, w = NB * 1024;
            acc[b][i] = red[o] + red[w + o] + red[2 * w + o] + red[3 * w + o];
        }
    if (slices > 1) {
        int32_t* mine = part + ((int64_t)tile * slices + sl) * NB * 1024;
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int i = 0; i < 16; i++)
                __hip_atomic_store(mine + b * 1024 + i * 64 + lane, acc[b][i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);   // the partial tile has reached the coherence point
        unsigned before = 0;
        if (lane == 0) before = __hip_atomic_fetch_add(counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        before = (unsigned)__builtin_amdgcn_readlane((int)before, 0);
        if ((int)before != slices - 1) return;   // not the last: the last one finishes the tile
        // every other slice's tile straight into LDS (device-coherent loads,
        // 1 KiB per instruction, all in flight at once), then the sums
        for (int z = 0, q = 0; z < slices; z++) {
            if (z == sl) continue;
            const int32_t* other = part + ((int64_t)tile * slices + z) * NB * 1024;
#pragma unroll
            for (int c = 0; c < NB * 4; c++)
                __builtin_amdgcn_global_load_lds((GlobalVoid*)(other + c * 256 + lane * 4),
                                                 (LdsVoid*)(red + (q * NB * 4 + c) * 256), 16, 0, kCoherentLoad);
            q++;
        }
        __builtin_amdgcn_s_waitcnt(0);
        for (int q = 0; q < slices - 1; q++)
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int i = 0; i < 16; i++) acc[b][i] += red[((q * NB + b) * 16 + i) * 64 + lane];
        if (lane == 0) __hip_atomic_store(counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const int n = n0 + col;
    if (n >= a.n) return;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int m = 8 * (i >> 2) + 4 * hi + (i & 3);
        if (m >= a.m) continue;
        const int64_t idx = (int64_t)m * a.n + n;
        if (EPI == EPI_RAW) {
            a.acc[idx] = acc[0][i];
            continue;
        }
        const double sx = a.as[m];
        const float v0 = (float)acc[0][i] * deq_mult(sx, a.ws[n]);
        if (EPI == EPI_GLU) {
            const float up = (float)acc[NB - 1][i] * deq_mult(sx, a.ws2[n]);
            a.y[idx] = tl_silu(v0) * up;
        } else if (EPI == EPI_DEQUANT_RES) {
            a.y[idx] = a.residual[idx] + v0;
        } else {
            a.y[idx] = v0;
        }
    }
}

// ---------------------------------------------------------------------------
// Q/K/V post-processing per row (GI:150-156, design_decisions A7/B2):
// RoPE on Q and K (TL:69-80), Q quantized at the row's own scale, K (post
// RoPE) and V quantized at the static per-layer/per-KV-head scales and
// appended to the KV cache at the row's position.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void qkv_post_kernel(const float* __restrict__ qkv, int32_t n_heads,
                                                       int32_t n_kv, RowMap rm,
                                                       const float* __restrict__ cosb,
                                                       const float* __restrict__ sinb, KvGeom kv,
                                                       int32_t layer, const float* __restrict__ kv_sk,
                                                       const float* __restrict__ kv_sv,
                                                       int8_t* __restrict__ q8,
                                                       double* __restrict__ q_scale,
                                                       float* __restrict__ q_rot_out, int32_t append_kv) {
    extern __shared__ __align__(16) float lds[];
    __shared__ float red[16];
    const int row = blockIdx.x, tid = threadIdx.x;
    const int D = n_heads * kHeadDim, KVD = n_kv * kHeadDim, W = D + 2 * KVD;   // multiples of 64
    float* v = lds;          // [W] inputs
    float* o = lds + W;      // [D + KVD] rotated q, k
    const float4* src = (const float4*)(qkv + (int64_t)row * W);
    for (int c = tid; c < W / 4; c += blockDim.x) ((float4*)v)[c] = src[c];
    __syncthreads();
    const int pos = rm.pos[row], seq = rm.seq[row];
    if (pos < 0 || pos >= kv.max_pos) return;   // a row outside the cache (uniform per workgroup)
    const float* cp = cosb + (int64_t)pos * kHeadDim;
    const float* sp = sinb + (int64_t)pos * kHeadDim;
    // four dimensions d .. d + 3 per step, all on one side of d = 32
    float mx = 0.0f;
    for (int c = tid; c < (D + KVD) / 4; c += blockDim.x) {
        const int d = (4 * c) & 63;
        const bool lo = d < 32;
        const float4 x = ((const float4*)v)[c];
        const float4 pr = ((const float4*)v)[lo ? c + 8 : c - 8];
        const float4 cc = *(const float4*)(cp + d), ss = *(const float4*)(sp + d);
        float4 r;
        r.x = (x.x * cc.x) + ((lo ? -pr.x : pr.x) * ss.x);
        r.y = (x.y * cc.y) + ((lo ? -pr.y : pr.y) * ss.y);
        r.z = (x.z * cc.z) + ((lo ? -pr.z : pr.z) * ss.z);
        r.w = (x.w * cc.w) + ((lo ? -pr.w : pr.w) * ss.w);
        ((float4*)o)[c] = r;
        if (4 * c < D) mx = fmaxf(mx, fmaxf(fmaxf(fabsf(r.x), fabsf(r.y)), fmaxf(fabsf(r.z), fabsf(r.w))));
    }
    mx = block_max(mx, red);  // includes the barrier that publishes o[]
    const double s = quant_scale(mx);
    // Q at the row's scale, four bytes per store; |q| <= max |q| keeps q y finite
    const RnDiv dq = rn_div_prep((float)s);
    auto qrow = [&](auto fast) {
        for (int c = tid; c < D / 4; c += blockDim.x) {
            const float4 r = ((const float4*)o)[c];
            ((unsigned*)(q8 + (int64_t)row * D))[c] = quant4<decltype(fast)::value>(r, dq);
            if (q_rot_out) ((float4*)(q_rot_out + (int64_t)row * D))[c] = r;
        }
    };
    if (dq.fast) qrow(std::true_type{});
    else qrow(std::false_type{});
    if (tid == 0) q_scale[row] = s;
    if (!append_kv) return;
    for (int i = tid; i < KVD; i += blockDim.x) {
        const int g = i >> 6, d = i & 63;
        const int64_t pl = kv.plane(seq, layer, g);
        kv.k[pl + KvGeom::k_off(pos, d)] = sat_i8(__builtin_rintf(__fdiv_rn(o[D + i], kv_sk[layer * n_kv + g])));
        kv.v[pl + KvGeom::v_off(pos, d)] = sat_i8(__builtin_rintf(__fdiv_rn(v[D + KVD + i], kv_sv[layer * n_kv + g])));
    }
}

// ---------------------------------------------------------------------------
// GQA attention over the INT8 KV cache, one workgroup per (row, KV head)
// covering the G = n_heads / n_kv query heads that share the KV head
// (gqa_router.sv:29).  For query position pos, keys 0..pos:
//   S = q8 . k8 (INT32, v_dot4), s = f32(S) * f32((s_q s_k) attn_scale)
//   softmax with the block-64 butterfly denominator, p8 = rne(127 p)
//   O = p8 . v8 (INT32), out = f32(O) * f32((1/127) s_v)
// ---------------------------------------------------------------------------
constexpr int kMaxGroup = 8;

__global__ __launch_bounds__(256) void attention_kernel(const int8_t* __restrict__ q8,
                                                        const double* __restrict__ q_scale,
                                                        int32_t n_heads, int32_t n_kv, RowMap rm,
                                                        KvGeom kv, int32_t layer,
                                                        const float* __restrict__ kv_sk,
                                                        const float* __restrict__ kv_sv,
                                                        double attn_scale, float* __restrict__ out,
                                                        AttnDebug dbg) {
    extern __shared__ float s_buf[];            // [G][tpad] scores then exps
    __shared__ int4 qs[kMaxGroup][4];           // q8 of the group's heads
    __shared__ float wmax[4][kMaxGroup];
    __shared__ float mrow[kMaxGroup], tot[kMaxGroup], scl[kMaxGroup];
    __shared__ int accs[4][kMaxGroup][64];

    const int g = blockIdx.x, row = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = n_heads / n_kv;
    const int pos = rm.pos[row], seq = rm.seq[row];
    if (pos < 0 || pos >= kv.max_pos) return;   // a row outside the cache (uniform per workgroup)
    const int T = pos + 1;
    const int tpad = (T + 63) & ~63;
    const int nblk = tpad >> 6;
    int8_t* p8 = (int8_t*)(s_buf + G * tpad);   // [G][tpad]
    float* bsum = (float*)(p8 + G * tpad);       // [G][nblk]

    const int D = n_heads * kHeadDim;
    const int8_t* qrow = q8 + (int64_t)row * D + (int64_t)g * G * kHeadDim;
    if (tid < G * 4) qs[tid >> 2][tid & 3] = ((const int4*)qrow)[tid];
    if (tid < G) {
        const float sk = kv_sk[layer * n_kv + g];
        scl[tid] = (float)((q_scale[row] * (double)sk) * attn_scale);
        if (dbg.score_scale && row == 0) dbg.score_scale[g * G + tid] = scl[tid];
    }
    const bool dbg_row = row == 0 && dbg.n_keys > 0;
    __syncthreads();

    const int64_t pl = kv.plane(seq, layer, g);
    const int8_t* kp = kv.k + pl;
    const int8_t* vp = kv.v + pl;

    // scores: lane <-> key within a block of 64
    float lmax[kMaxGroup];
#pragma unroll
    for (int h = 0; h < kMaxGroup; h++) lmax[h] = -INFINITY;
    for (int b = wave; b < nblk; b += 4) {
        const int t = b * 64 + lane;
        if (t < T) {
            const int8_t* kb = kp + (int64_t)b * 4096 + lane * 16;
            const int4 k0 = *(const int4*)(kb);
            const int4 k1 = *(const int4*)(kb + 1024);
            const int4 k2 = *(const int4*)(kb + 2048);
            const int4 k3 = *(const int4*)(kb + 3072);
#pragma unroll
            for (int h = 0; h < kMaxGroup; h++) {
                if (h < G) {
                    int S = sdot4x4(k0, qs[h][0], 0);
                    S = sdot4x4(k1, qs[h][1], S);
                    S = sdot4x4(k2, qs[h][2], S);
                    S = sdot4x4(k3, qs[h][3], S);
                    const float sv = (float)S * scl[h];
                    s_buf[h * tpad + t] = sv;
                    if (dbg_row && dbg.scores && t >= dbg.key0 && t < dbg.key0 + dbg.n_keys)
                        dbg.scores[(int64_t)(g * G + h) * dbg.n_keys + (t - dbg.key0)] = S;
                    lmax[h] = fmaxf(lmax[h], sv);
                }
            }
        }
    }
#pragma unroll
    for (int h = 0; h < kMaxGroup; h++) {
        if (h < G) {
            const float m = wave_max_f32(lmax[h]);
            if (lane == 0) wmax[wave][h] = m;
        }
    }
    __syncthreads();
    if (tid < G) {
        float m = wmax[0][tid];
        for (int w = 1; w < 4; w++) m = fmaxf(m, wmax[w][tid]);
        mrow[tid] = m;
    }
    __syncthreads();

    // exponentials and per-block butterfly sums
    for (int b = wave; b < nblk; b += 4) {
        const int t = b * 64 + lane;
#pragma unroll
        for (int h = 0; h < kMaxGroup; h++) {
            if (h < G) {
                float e = 0.0f;
                if (t < T) {
                    e = tl_expf(s_buf[h * tpad + t] - mrow[h]);
                    s_buf[h * tpad + t] = e;
                }
                const float bs = wave_butterfly_sum(e);
                if (lane == 0) bsum[h * nblk + b] = bs;
            }
        }
    }
    __syncthreads();
    if (tid < G) {
        const float total = ordered_sum(bsum + tid * nblk, nblk);
        tot[tid] = total;
    }
    __syncthreads();

    // INT8 probabilities (EX:870-873), zero beyond the last key
    for (int t = tid; t < tpad; t += blockDim.x) {
        for (int h = 0; h < G; h++) {
            int8_t pq = 0;
            if (t < T) {
                float pr = __builtin_rintf(__fdiv_rn(s_buf[h * tpad + t], tot[h]) * 127.0f);
                pr = pr < 0.0f ? 0.0f : (pr > 127.0f ? 127.0f : pr);
                pq = (int8_t)(int)pr;
            }
            p8[h * tpad + t] = pq;
            if (dbg_row && dbg.probs && t >= dbg.key0 && t < dbg.key0 + dbg.n_keys)
                dbg.probs[(int64_t)(g * G + h) * dbg.n_keys + (t - dbg.key0)] = pq;
        }
    }
    __syncthreads();

    // O = P8 . V8: lane d reads dimension d of 16 consecutive keys (one
    // coalesced 1 KiB load per wavefront) and dots it with each head's 16
    // probabilities
    int o[kMaxGroup];
#pragma unroll
    for (int h = 0; h < kMaxGroup; h++) o[h] = 0;
    const int ngrp = tpad >> 4;
    for (int c = wave; c < ngrp; c += 4) {
        const int4 vv = *(const int4*)(vp + (int64_t)c * 1024 + lane * 16);
#pragma unroll
        for (int h = 0; h < kMaxGroup; h++)
            if (h < G) o[h] = sdot4x4(vv, *(const int4*)(p8 + h * tpad + c * 16), o[h]);
    }
#pragma unroll
    for (int h = 0; h < kMaxGroup; h++)
        if (h < G) accs[wave][h][lane] = o[h];
    __syncthreads();
    const float pv_mult = deq_mult(1.0 / 127.0, kv_sv[layer * n_kv + g]);
    for (int i = tid; i < G * 64; i += blockDim.x) {
        const int h = i >> 6, d = i & 63;
        const int O = accs[0][h][d] + accs[1][h][d] + accs[2][h][d] + accs[3][h][d];
        out[(int64_t)row * D + (int64_t)(g * G + h) * kHeadDim + d] = (float)O * pv_mult;
    }
}


// ---------------------------------------------------------------------------
// prefill attention on i8 MFMA (v_mfma_i32_32x32x32_i8), same arithmetic as
// attention_kernel: one workgroup (4 wavefronts) per (query head, tile of 32
// consecutive rows of one sequence at positions pos0 + r).  The INT8 cache
// layouts are the MFMA operand fragments: lane l of a K fragment holds 16
// dimensions of key l % 32 (one 16-byte chunk of the K plane), lane l of a V
// fragment 16 keys of dimension l % 32 (one chunk of the V plane).  In the
// 32 x 32 output lane l, register i holds row 8 (i / 4) + 4 (l / 32) + i % 4
// and key (or dimension) l % 32.
//   pass A  S = Q K^T per 32-key tile, row maxima over each row's keys
//   pass B  exponentials; a 64-key block is two tiles, so the block-64
//           butterfly is the sum of the two tiles' values (distance 32) and
//           then lane distances 16 .. 1 -- the order of the decode kernels;
//           row totals in block order
//   pass C  p8 = rne(127 e / total) into LDS (rows x keys)
//   pass D  O = P8 . V per 32-key chunk, integer partials added in LDS
// Scores are recomputed per pass (K is an L2 hit), so LDS does not grow with
// the context beyond the INT8 probabilities.
// ---------------------------------------------------------------------------
struct AttnTileArgs {
    const int8_t* q8;        // [rows][D]
    const double* q_scale;   // [rows]
    int32_t n_heads, n_kv, rows, seq, pos0, layer;
    KvGeom kv;
    const float* kv_sk;
    const float* kv_sv;
    double attn_scale;
    float* out;              // [rows][D]
    const float* qf;         // or rotated Q in float32 [rows][D], quantized here
    const unsigned* qmax;    // with qf: max|q| of each row as float bits [rows][kQmaxStride]
};

// Q fragments of a tile lane (row r, head h, K halves hi * 16 .. + 16 and
// 32 + hi * 16 .. + 16), in three steps around the workgroup barrier that
// follows the K and V loads.  From q8 the fragments are loaded directly.
// From float32 Q the workgroup quantizes the tile once: thread t takes row
// t / 8, dimensions 8 (t % 8) .. + 8, at the row's scale exactly as
// qkv_post_kernel does (quant_scale of the row maximum, the correctly rounded
// division of rn_div_prep / quant4; the fast form only when every lane's
// divisor allows it, both give RN(q / s)), into a 32 x 64 byte LDS tile that
// every wavefront then reads its fragments from.
struct TileQ {
    v4i qa0, qa1;
    float4 x0, x1;
    unsigned mx;
};

TL_DEV void tile_q_load(const AttnTileArgs& p, int r0, int nr, int h, int col, int hi, TileQ& q) {
    const int D = p.n_heads * kHeadDim;
    if (!p.qf) {
        const int8_t* qrow = p.q8 + (int64_t)(r0 + min(col, nr - 1)) * D + h * kHeadDim + hi * 16;
        q.qa0 = ld16(qrow);
        q.qa1 = ld16(qrow + 32);
        return;
    }
    const int r = r0 + min((int)threadIdx.x >> 3, nr - 1);   // rows past the tile's last: a stand-in, never stored
    const float4* qr = (const float4*)(p.qf + (int64_t)r * D + h * kHeadDim + (threadIdx.x & 7) * 8);
    q.x0 = qr[0];
    q.x1 = qr[1];
    q.mx = p.qmax[(int64_t)r * kQmaxStride];
}

// before the barrier: quantize this thread's 8 values into qs8 ([32][64])
TL_DEV void tile_q_quantize(const AttnTileArgs& p, TileQ& q, int8_t* qs8) {
    if (!p.qf) return;
    RnDiv dq;
    dq.b = (float)quant_scale(__uint_as_float(q.mx));
    dq.y = __fdiv_rn(1.0f, dq.b);
    dq.fast = __all(fabsf(dq.b) >= 0x1p-64f && fabsf(dq.b) <= 0x1p64f);
    const unsigned u0 = dq.fast ? quant4<true>(q.x0, dq) : quant4<false>(q.x0, dq);
    const unsigned u1 = dq.fast ? quant4<true>(q.x1, dq) : quant4<false>(q.x1, dq);
    *(uint2*)(qs8 + threadIdx.x * 8) = make_uint2(u0, u1);
}

// after the barrier: the lane's fragments out of qs8
TL_DEV void tile_q_frags(const AttnTileArgs& p, const int8_t* qs8, int col, int hi, TileQ& q) {
    if (!p.qf) return;
    q.qa0 = *(const v4i*)(qs8 + col * 64 + hi * 16);
    q.qa1 = *(const v4i*)(qs8 + col * 64 + 32 + hi * 16);
}

// the row's Q scale (GI:36-42) for the score dequantization
TL_DEV double tile_q_scale(const AttnTileArgs& p, int r) {
    return p.qf ? quant_scale(__uint_as_float(p.qmax[(int64_t)r * kQmaxStride])) : p.q_scale[r];
}

__global__ __launch_bounds__(256) void attention_tile_kernel(AttnTileArgs p) {
    extern __shared__ __align__(16) int8_t tile_lds[];
    __shared__ __align__(16) int8_t qs8[32 * 64];   // Q quantized by the workgroup (float32 Q input)
    __shared__ float scl[32], mrow[32], tot[32];
    __shared__ float wmax[4][32];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int col = lane & 31, hi = lane >> 5;
    const int h = blockIdx.x, r0 = (gridDim.y - 1 - blockIdx.y) * 32;   // the longest (last) tiles dispatch first
    const int G = p.n_heads / p.n_kv, g = h / G;
    const int nr = min(32, p.rows - r0);
    const int pos_first = p.pos0 + r0;
    const int T = pos_first + nr;                  // the tile's last row sees keys 0 .. T - 1
    const int tpad = (T + 63) & ~63, nblk = tpad >> 6;
    int8_t* p8 = tile_lds;                         // [32][tpad]
    float* bsum = (float*)(tile_lds + 32 * tpad);  // [32][nblk]
    int* accs = (int*)(bsum + 32 * nblk);          // [32][64]
    const int D = p.n_heads * kHeadDim;
    const int64_t pl = p.kv.plane(p.seq, p.layer, g);
    const int8_t* kp = p.kv.k + pl;
    const int8_t* vp = p.kv.v + pl;
    const float sk = p.kv_sk[p.layer * p.n_kv + g], sv = p.kv_sv[p.layer * p.n_kv + g];

    // Q fragments (rows past the tile's last read a stand-in, never stored)
    TileQ tq;
    tile_q_load(p, r0, nr, h, col, hi, tq);
    if (tid < 32) scl[tid] = (float)((tile_q_scale(p, r0 + min(tid, nr - 1)) * (double)sk) * p.attn_scale);
    for (int e = tid; e < 32 * 64; e += 256) accs[e] = 0;
    tile_q_quantize(p, tq, qs8);
    __syncthreads();
    tile_q_frags(p, qs8, col, hi, tq);
    const v4i qa0 = tq.qa0, qa1 = tq.qa1;
    float rs[16];
    int rpos[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int r = 8 * (i >> 2) + 4 * hi + (i & 3);
        rs[i] = scl[r];
        rpos[i] = pos_first + r;
    }
    auto scores = [&](int kt) {
        const int t = kt * 32 + col;
        const int8_t* kb = kp + (int64_t)(t >> 6) * 4096 + hi * 1024 + (t & 63) * 16;
        const v4i k0 = ld16(kb), k1 = ld16(kb + 2048);
        v16i acc = {};
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(qa0, k0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(qa1, k1, acc, 0, 0, 0);
        return acc;
    };

    // pass A: row maxima
    float mx[16];
#pragma unroll
    for (int i = 0; i < 16; i++) mx[i] = -INFINITY;
    for (int b = wave; b < nblk; b += 4) {
#pragma unroll
        for (int half = 0; half < 2; half++) {
            const int kt = 2 * b + half, t = kt * 32 + col;
            const v16i S = scores(kt);
#pragma unroll
            for (int i = 0; i < 16; i++)
                if (t <= rpos[i]) mx[i] = fmaxf(mx[i], (float)S[i] * rs[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
        float v = mx[i];
        v = half_max_f32(v);
        if (col == 0) wmax[wave][8 * (i >> 2) + 4 * hi + (i & 3)] = v;
    }
    __syncthreads();
    if (tid < 32) mrow[tid] = fmaxf(fmaxf(wmax[0][tid], wmax[1][tid]), fmaxf(wmax[2][tid], wmax[3][tid]));
    __syncthreads();
    float m[16];
#pragma unroll
    for (int i = 0; i < 16; i++) m[i] = mrow[8 * (i >> 2) + 4 * hi + (i & 3)];

    // pass B: block sums
    for (int b = wave; b < nblk; b += 4) {
        const v16i S0 = scores(2 * b), S1 = scores(2 * b + 1);
        const int t0 = 64 * b + col, t1 = t0 + 32;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float e0 = t0 <= rpos[i] ? tl_expf((float)S0[i] * rs[i] - m[i]) : 0.0f;
            const float e1 = t1 <= rpos[i] ? tl_expf((float)S1[i] * rs[i] - m[i]) : 0.0f;
            float v = e0 + e1;
            v = half_butterfly_sum(v);
            if (col == 0) bsum[(8 * (i >> 2) + 4 * hi + (i & 3)) * nblk + b] = v;
        }
    }
    __syncthreads();
    if (tid < 32) {
        const float total = ordered_sum(bsum + tid * nblk, nblk);
        tot[tid] = total;
    }
    __syncthreads();

    // pass C: INT8 probabilities (zero past each row's last key): exponential
    // / total correctly rounded, from each row's reciprocal and two residual
    // corrections (e <= 1 <= total keeps e y finite; every total lies in
    // [1, keys], the quotient's range, which the wave vote confirms)
    float ty[16], tv[16];
    bool in_range = true;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        tv[i] = tot[8 * (i >> 2) + 4 * hi + (i & 3)];
        ty[i] = __fdiv_rn(1.0f, tv[i]);
        in_range = in_range && fabsf(tv[i]) >= 0x1p-64f && fabsf(tv[i]) <= 0x1p64f;
    }
    const bool fast = __all(in_range);
    for (int b = wave; b < nblk; b += 4) {
#pragma unroll
        for (int half = 0; half < 2; half++) {
            const int kt = 2 * b + half, t = kt * 32 + col;
            const v16i S = scores(kt);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int r = 8 * (i >> 2) + 4 * hi + (i & 3);
                int8_t pq = 0;
                if (t <= rpos[i]) {
                    const float e = tl_expf((float)S[i] * rs[i] - m[i]);
                    const float q = fast ? rn_div_fast(e, RnDiv{tv[i], ty[i], true}) : __fdiv_rn(e, tv[i]);
                    float pr = __builtin_rintf(q * 127.0f);
                    pr = pr < 0.0f ? 0.0f : (pr > 127.0f ? 127.0f : pr);
                    pq = (int8_t)(int)pr;
                }
                p8[r * tpad + t] = pq;
            }
        }
    }
    __syncthreads();

    // pass D: O = P8 . V
    v16i o0 = {}, o1 = {};
    for (int kc = wave; kc < tpad / 32; kc += 4) {
        const v4i a = *(const v4i*)(p8 + col * tpad + kc * 32 + hi * 16);
        const int8_t* vb = vp + (int64_t)(kc * 2 + hi) * 1024 + col * 16;
        const v4i b0 = ld16(vb), b1 = ld16(vb + 512);
        o0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b0, o0, 0, 0, 0);
        o1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b1, o1, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int r = 8 * (i >> 2) + 4 * hi + (i & 3);
        atomicAdd(&accs[r * 64 + col], o0[i]);
        atomicAdd(&accs[r * 64 + 32 + col], o1[i]);
    }
    __syncthreads();
    const float pv_mult = deq_mult(1.0 / 127.0, sv);
    for (int e = tid; e < 32 * 64; e += 256) {
        const int r = e >> 6, d = e & 63;
        if (r < nr) p.out[(int64_t)(r0 + r) * D + (int64_t)h * kHeadDim + d] = (float)accs[e] * pv_mult;
    }
}

// ---------------------------------------------------------------------------
// standalone element-wise ops (operator surface of TL)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rope_kernel(float* __restrict__ v, int32_t n_heads,
                                                   const int32_t* __restrict__ pos,
                                                   const float* __restrict__ cosb,
                                                   const float* __restrict__ sinb) {
    extern __shared__ float lds[];
    const int row = blockIdx.x, n = n_heads * kHeadDim;
    float* r = v + (int64_t)row * n;
    for (int i = threadIdx.x; i < n; i += blockDim.x) lds[i] = r[i];
    __syncthreads();
    const float* cp = cosb + (int64_t)pos[row] * kHeadDim;
    const float* sp = sinb + (int64_t)pos[row] * kHeadDim;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int d = i & 63;
        const float rot = d < 32 ? -lds[i + 32] : lds[i - 32];
        r[i] = (lds[i] * cp[d]) + (rot * sp[d]);
    }
}

// softmax of each row with the block-64 butterfly denominator
__global__ __launch_bounds__(256) void softmax_rows_kernel(const float* __restrict__ x, int32_t n,
                                                           float* __restrict__ p) {
    extern __shared__ float bs[];
    __shared__ float red[16];
    __shared__ float mtot[2];
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* xr = x + (int64_t)row * n;
    float* pr = p + (int64_t)row * n;
    float mx = -INFINITY;
    for (int i = tid; i < n; i += blockDim.x) mx = fmaxf(mx, xr[i]);
    mx = wave_max_f32(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    if (tid == 0) {
        float m = red[0];
        for (int w = 1; w < (int)(blockDim.x >> 6); w++) m = fmaxf(m, red[w]);
        mtot[0] = m;
    }
    __syncthreads();
    const float m = mtot[0];
    const int nblk = (n + 63) >> 6;
    for (int b = wave; b < nblk; b += blockDim.x >> 6) {
        const int t = b * 64 + lane;
        float e = 0.0f;
        if (t < n) {
            e = tl_expf(xr[t] - m);
            pr[t] = e;
        }
        const float s = wave_butterfly_sum(e);
        if (lane == 0) bs[b] = s;
    }
    __syncthreads();
    if (tid == 0) {
        const float total = ordered_sum(bs, nblk);
        mtot[1] = total;
    }
    __syncthreads();
    const float total = mtot[1];
    for (int i = tid; i < n; i += blockDim.x) pr[i] = __fdiv_rn(pr[i], total);
}

// GI:45-46 (+ bias, GI:72-73): y = f32(acc) * m (+ b[col]); the multiplier m
// = f32(input_scale * weight_scale) is formed on the host in double, as the
// golden forms its Python-float product before the float32 multiply.  Without
// a bias nothing is added (adding +0 would turn -0 into +0).
__global__ __launch_bounds__(256) void dequant_i32_kernel(const int32_t* __restrict__ acc, int64_t n, int32_t cols,
                                                          float m, const float* __restrict__ bias,
                                                          float* __restrict__ y) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float v = (float)acc[i] * m;
        y[i] = bias ? v + bias[i % cols] : v;
    }
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ g,
                                                       const float* __restrict__ u, int64_t n,
                                                       float* __restrict__ y) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = u ? tl_silu(g[i]) * u[i] : tl_silu(g[i]);
}

// embedding row of the INT8 table: x = f32(e8[tok]) * s_e[tok]
// (an id outside [0, vocab) yields a zero row instead of an out-of-bounds read)
__global__ __launch_bounds__(256) void embed_kernel(const int32_t* __restrict__ tokens, int32_t d,
                                                    int32_t vocab, const int8_t* __restrict__ emb,
                                                    const float* __restrict__ emb_s,
                                                    float* __restrict__ x) {
    const int row = blockIdx.x;
    const int tok = tokens[row];
    if (tok < 0 || tok >= vocab) {
        for (int i = threadIdx.x; i < d; i += blockDim.x) x[(int64_t)row * d + i] = 0.0f;
        return;
    }
    const int8_t* e = emb + (int64_t)tok * d;
    const float s = emb_s[tok];
    for (int i = threadIdx.x; i < d; i += blockDim.x) x[(int64_t)row * d + i] = (float)e[i] * s;
}

__global__ void reset_keys_kernel(unsigned long long* keys, int32_t n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) keys[i] = 0ull;
}

// after the LM head: decode each row's argmax key into the current token,
// append it to the row's output list, advance the cursor, clear the key.
// With one row (single = one wavefront): the LM head may have left one key
// per workgroup (wg_keys, folded here), and with x the new token's embedding
// and position are written for the next step (what embed_step_kernel does).
// With nx.stopped, a stopped sequence records nothing; the token that stopped
// it is embedded again at the unchanged cursor.
__global__ __launch_bounds__(64) void finalize_tokens_kernel(unsigned long long* keys, int32_t rows,
                                                             int32_t* token_cur, int32_t* tokens_out,
                                                             int32_t out_stride, int32_t* n_gen, int32_t* cursor,
                                                             float* best_logit, int32_t advance,
                                                             const unsigned long long* wg_keys, int32_t n_wg,
                                                             EmbedNext nx) {
    const WaveStamp stamp(nx.ts, blockIdx.x);
    const bool single = n_wg > 0 || nx.x != nullptr;
    const int r = single ? 0 : blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    // every independent load first, so the step pays one memory round trip
    // before the embedding gather: the stop flag, this row's key and state,
    // and the first kFinUnroll x 64 workgroup keys.  Every lane reads the flag
    // and the key before lane 0 may write them.
    constexpr int kFinUnroll = 16;
    const int32_t stop_v = (single && nx.stopped != nullptr) ? *nx.stopped : 0;
    const int32_t abort_v = (single && nx.abort_word != nullptr)
                                ? __hip_atomic_load(nx.abort_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM)
                                : 0;
    const unsigned long long key_r = keys[r];
    const int32_t tok_r = token_cur[r], cur_r = cursor[r], gen_r = n_gen[r];
    const int32_t eos = (single && nx.eos) ? *nx.eos : -1;
    unsigned long long wk[kFinUnroll];
#pragma unroll
    for (int j = 0; j < kFinUnroll; j++) {
        const int i = threadIdx.x + 64 * j;
        wk[j] = i < n_wg ? wg_keys[i] : 0ull;
    }
    // a host abort outranks EOS (stop_condition_unit.sv:26-28): a step that
    // sees it records nothing, even the token that would have been the EOS
    const bool halted = stop_v != 0 || abort_v != 0;
    int32_t tok, cur;
    if (halted) {
        tok = tok_r;
        cur = cur_r;
        if (threadIdx.x == 0) {
            keys[r] = 0ull;
            if (nx.x) *nx.row_pos = cur;
            if (stop_v == 0 && nx.stopped) {
                *nx.stopped = 2;
                if (nx.stop_host) __hip_atomic_store(nx.stop_host, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
        }
    } else {
        unsigned long long fold = 0;
        if (n_wg > 0) {
#pragma unroll
            for (int j = 0; j < kFinUnroll; j++) fold = max_u64(fold, wk[j]);
            for (int i = threadIdx.x + 64 * kFinUnroll; i < n_wg; i += 64) fold = max_u64(fold, wg_keys[i]);
            fold = wave_max_u64(fold);
        }
        const unsigned long long k = max_u64(key_r, fold);
        tok = key_index(k);
        cur = cur_r + advance;
        if (!single || threadIdx.x == 0) {
            token_cur[r] = tok;
            const int32_t i = gen_r;
            if (i >= 0 && i < out_stride) {
                if (tokens_out) tokens_out[(int64_t)r * out_stride + i] = tok;
                if (best_logit) best_logit[(int64_t)r * out_stride + i] = key_logit(k);
            }
            n_gen[r] = i + 1;
            cursor[r] = cur;
            keys[r] = 0ull;
            if (nx.x) *nx.row_pos = cur;
            if (single && nx.stopped && eos >= 0 && tok == eos) {
                *nx.stopped = 1;
                if (nx.stop_host) __hip_atomic_store(nx.stop_host, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
        }
    }
    if (nx.x) {
        const bool ok = tok >= 0 && tok < nx.vocab;   // otherwise a zero row, as embed_step_kernel
        const int t = ok ? tok : 0;
        const int8_t* e = nx.emb + (int64_t)t * nx.d;
        const float sc = nx.emb_s[t];
        if (nx.d % 16 == 0) {   // 16 bytes in, four float4 out per step (rows are 16-byte aligned)
            for (int i = 16 * threadIdx.x; i < nx.d; i += 16 * 64) {
                const v4i w = *(const v4i*)(e + i);
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    float4 f;
                    f.x = ok ? (float)(int8_t)(w[q] & 0xFF) * sc : 0.0f;
                    f.y = ok ? (float)(int8_t)((w[q] >> 8) & 0xFF) * sc : 0.0f;
                    f.z = ok ? (float)(int8_t)((w[q] >> 16) & 0xFF) * sc : 0.0f;
                    f.w = ok ? (float)(int8_t)((w[q] >> 24) & 0xFF) * sc : 0.0f;
                    *(float4*)(nx.x + i + 4 * q) = f;
                }
            }
        } else {
            for (int i = threadIdx.x; i < nx.d; i += 64) nx.x[i] = ok ? (float)e[i] * sc : 0.0f;
        }
    }
}

// requantize_unit.sv:39-115: y[i] = clamp(rne16(acc[i] * m[i / lanes_per_scale]))
// with m unsigned Q16.16 (the 64-bit product is exact), round half to even on
// the 16 fraction bits of the magnitude, then +-127 (or [0, 127] when
// nonnegative_only); lanes at or past `active` give 0 (the unit's
// elem_count).
__global__ __launch_bounds__(256) void requant_q16_kernel(const int32_t* __restrict__ acc,
                                                          const uint32_t* __restrict__ scale, int32_t n,
                                                          int32_t active, int32_t lanes_per_scale,
                                                          int32_t nonnegative_only, int8_t* __restrict__ y) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (i >= active) {
        y[i] = 0;
        return;
    }
    const long long prod = (long long)acc[i] * (long long)scale[i / lanes_per_scale];
    const unsigned long long mag = prod < 0 ? (unsigned long long)(-prod) : (unsigned long long)prod;
    unsigned long long q = mag >> 16;
    const unsigned rem = (unsigned)(mag & 0xFFFFull);
    if (rem > 0x8000u || (rem == 0x8000u && (q & 1ull))) q += 1;
    long long r = prod < 0 ? -(long long)q : (long long)q;
    const long long lo = nonnegative_only ? 0 : -127;
    r = r > 127 ? 127 : (r < lo ? lo : r);
    y[i] = (int8_t)r;
}

hipError_t launch_requant_q16(hipStream_t s, const int32_t* acc, const uint32_t* scale, int32_t n, int32_t active,
                              int32_t lanes_per_scale, int32_t nonnegative_only, int8_t* y) {
    if (n <= 0) return hipSuccess;
    if (lanes_per_scale < 1) return hipErrorInvalidValue;
    TL_KLAUNCH(requant_q16_kernel, dim3((n + 255) / 256), dim3(256), 0, s, acc, scale, n, active, lanes_per_scale,
               nonnegative_only, y);
    return hipGetLastError();
}

// causal_mask_unit.sv:37-54 (EX:1157-1184) over a tile of INT32 scores
// [rows][cols]: element (r, c) keeps its score when r < query_row_count,
// c < key_col_count and key_pos_base + c <= query_pos_base + r; other
// elements of active rows become MASK_NEG_INF, rows past query_row_count 0
constexpr int32_t kMaskNegInf = -1000000000;   // tinyllama_pkg.sv MASK_NEG_INF

__global__ __launch_bounds__(256) void causal_mask_i32_kernel(const int32_t* __restrict__ s, int64_t total,
                                                              int32_t cols, int32_t qb, int32_t kb, int32_t qrc,
                                                              int32_t kcc, int32_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int32_t r = (int32_t)(i / cols), c = (int32_t)(i % cols);
    int32_t v = 0;
    if (r < qrc) {
        const bool allow = c < kcc && (int64_t)kb + c <= (int64_t)qb + r;
        v = allow ? s[i] : kMaskNegInf;
    }
    out[i] = v;
}

hipError_t launch_causal_mask_i32(hipStream_t s, const int32_t* scores, int32_t rows, int32_t cols, int32_t qb,
                                  int32_t kb, int32_t qrc, int32_t kcc, int32_t* out) {
    const int64_t total = (int64_t)rows * cols;
    if (total <= 0) return hipSuccess;
    TL_KLAUNCH(causal_mask_i32_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, scores, total, cols, qb,
               kb, qrc, kcc, out);
    return hipGetLastError();
}

// rope_unit.sv:73-127 (EX:684-732) INT8 RoPE: the Q16.16 cos / sin of the
// row's position are the float32 table (build_rope_cache) times 2^16 rounded
// to nearest even, as EX:158-161 forms the ROM; dimension d < 32 gives
// rne16(x_d c - x_{d+32} s), d >= 32 rne16(x_d c + x_{d-32} s), both
// saturated to +-127.  Positions outside the table are clamped to it (the
// operator checks host positions before the launch).
__global__ __launch_bounds__(256) void rope_q16_kernel(const int8_t* __restrict__ x, int64_t total, int32_t width,
                                                       const int32_t* __restrict__ pos, const float* __restrict__ cosb,
                                                       const float* __restrict__ sinb, int32_t n_pos,
                                                       int8_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int64_t r = i / width;
    const int32_t e = (int32_t)(i % width), d = e & (kHeadDim - 1);
    const int32_t p = min(max(pos[r], 0), n_pos - 1);
    const int32_t cq = (int32_t)__builtin_rintf(cosb[(int64_t)p * kHeadDim + d] * 65536.0f);
    const int32_t sq = (int32_t)__builtin_rintf(sinb[(int64_t)p * kHeadDim + d] * 65536.0f);
    const bool lower = d < kHeadDim / 2;
    const int32_t curr = x[i], pair = x[lower ? i + kHeadDim / 2 : i - kHeadDim / 2];
    const long long sum = lower ? (long long)curr * cq - (long long)pair * sq : (long long)curr * cq + (long long)pair * sq;
    const unsigned long long mag = sum < 0 ? (unsigned long long)(-sum) : (unsigned long long)sum;
    unsigned long long q = mag >> 16;
    const unsigned rem = (unsigned)(mag & 0xFFFFull);
    if (rem > 0x8000u || (rem == 0x8000u && (q & 1ull))) q += 1;
    long long v = sum < 0 ? -(long long)q : (long long)q;
    v = v > 127 ? 127 : (v < -127 ? -127 : v);
    out[i] = (int8_t)v;
}

hipError_t launch_rope_q16(hipStream_t s, const int8_t* x, int32_t rows, int32_t n_heads, const int32_t* pos,
                           const float* cosb, const float* sinb, int32_t n_pos, int8_t* out) {
    const int64_t total = (int64_t)rows * n_heads * kHeadDim;
    if (total <= 0) return hipSuccess;
    TL_KLAUNCH(rope_q16_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, x, total, n_heads * kHeadDim,
               pos, cosb, sinb, n_pos, out);
    return hipGetLastError();
}

// argmax_reduction.sv:47-93 over INT32 logits: the greatest value, the lowest
// index among equal ones.  Each value becomes a 64-bit key (the value's
// order-preserving bits above, the complemented index below); workgroups
// fold theirs with one atomicMax into *key (zero before the launch)
__global__ __launch_bounds__(256) void argmax_i32_kernel(const int32_t* __restrict__ v, int32_t n,
                                                         unsigned long long* __restrict__ key) {
    __shared__ unsigned long long wbest[4];
    unsigned long long best = 0;
    for (int32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const unsigned u = (unsigned)v[i] ^ 0x80000000u;
        best = max_u64(best, ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (unsigned)i));
    }
    best = wave_max_u64(best);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) wbest[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned long long b = max_u64(max_u64(wbest[0], wbest[1]), max_u64(wbest[2], wbest[3]));
        atomicMax(key, b);
    }
}

hipError_t launch_argmax_i32(hipStream_t s, const int32_t* v, int32_t n, unsigned long long* key) {
    if (n <= 0) return hipErrorInvalidValue;
    TL_KLAUNCH(reset_keys_kernel, dim3(1), dim3(64), 0, s, key, 1);
    const int grid = std::min(256, (n + 255) / 256);
    TL_KLAUNCH(argmax_i32_kernel, dim3(grid), dim3(256), 0, s, v, n, key);
    return hipGetLastError();
}

// argmax of each logits row (one workgroup per row) into its key slot
__global__ __launch_bounds__(256) void argmax_rows_kernel(const float* __restrict__ logits, int32_t n,
                                                          unsigned long long* __restrict__ keys) {
    __shared__ unsigned long long wbest[4];
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* lr = logits + (int64_t)row * n;
    unsigned long long best = 0;
    // eight loads in flight per thread (the max of the keys is order-free)
    for (int i0 = tid; i0 < n; i0 += 8 * blockDim.x) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = lr[min(i0 + j * (int)blockDim.x, n - 1)];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int i = i0 + j * (int)blockDim.x;
            if (i < n) {
                const unsigned long long k = argmax_key(v[j], i);
                best = k > best ? k : best;
            }
        }
    }
    best = wave_max_u64(best);
    if (lane == 0) wbest[wave] = best;
    __syncthreads();
    if (tid == 0) {
        unsigned long long b = wbest[0];
        for (int i = 1; i < 4; i++) b = wbest[i] > b ? wbest[i] : b;
        keys[row] = b;
    }
}

// the best of the per-tile keys [tiles][rows] of each row (one workgroup per
// row; the max of the keys is order-free)
__global__ __launch_bounds__(256) void argmax_tiles_kernel(const unsigned long long* __restrict__ part, int32_t tiles,
                                                           int32_t rows, unsigned long long* __restrict__ keys) {
    __shared__ unsigned long long wbest[4];
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    unsigned long long best = 0;
    for (int t0 = tid; t0 < tiles; t0 += 8 * blockDim.x) {
        unsigned long long v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int t = t0 + j * (int)blockDim.x;
            v[j] = part[(int64_t)min(t, tiles - 1) * rows + row];
        }
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (t0 + j * (int)blockDim.x < tiles) best = v[j] > best ? v[j] : best;
    }
    best = wave_max_u64(best);
    if (lane == 0) wbest[wave] = best;
    __syncthreads();
    if (tid == 0) {
        unsigned long long b = wbest[0];
        for (int i = 1; i < 4; i++) b = wbest[i] > b ? wbest[i] : b;
        keys[row] = b;
    }
}

hipError_t launch_argmax_tiles(hipStream_t s, const unsigned long long* part, int32_t tiles, int32_t rows,
                               unsigned long long* keys) {
    if (rows <= 0 || tiles <= 0) return hipErrorInvalidValue;
    TL_KLAUNCH(argmax_tiles_kernel, dim3(rows), dim3(256), 0, s, part, tiles, rows, keys);
    return hipGetLastError();
}

// batched decode: the position of each row is its sequence's cursor
__global__ void step_rows_kernel(const int32_t* seq_of_row, int32_t rows, const int32_t* cursor,
                                 int32_t* row_pos) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r < rows) row_pos[r] = cursor[seq_of_row[r]];
}

// logical [n][64] rows <-> cache plane layout
__global__ void kv_scatter_kernel(KvGeom kv, int64_t pl, int32_t t0, int32_t n,
                                  const int8_t* __restrict__ k_rows, const int8_t* __restrict__ v_rows) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)n * kHeadDim) return;
    const int t = t0 + (int)(i >> 6), d = (int)(i & 63);
    if (k_rows) kv.k[pl + KvGeom::k_off(t, d)] = k_rows[i];
    if (v_rows) kv.v[pl + KvGeom::v_off(t, d)] = v_rows[i];
}

__global__ void kv_gather_kernel(KvGeom kv, int64_t pl, int32_t t0, int32_t n,
                                 int8_t* __restrict__ k_rows, int8_t* __restrict__ v_rows) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)n * kHeadDim) return;
    const int t = t0 + (int)(i >> 6), d = (int)(i & 63);
    if (k_rows) k_rows[i] = kv.k[pl + KvGeom::k_off(t, d)];
    if (v_rows) v_rows[i] = kv.v[pl + KvGeom::v_off(t, d)];
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
bool make_pw_plan(int32_t n, PwPlan* plan) {
    if (n < 8) return false;
    int32_t len = n, leaves = 1;
    while (len > 128) {
        if (len % 2 != 0 || (len / 2) % 8 != 0) return false;
        len /= 2;
        leaves *= 2;
    }
    if (len % 8 != 0) return false;
    plan->leaf_len = len;
    plan->n_leaves = leaves;
    return true;
}

static inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

hipError_t launch_rmsnorm_quant(hipStream_t s, const float* x, const float* g, int32_t rows,
                                int32_t n, float eps, PwPlan plan, float* y, int8_t* q,
                                double* scales, bool packed, const L2Prefetch* pf) {
    if (rows <= 0) return hipSuccess;
    if (!y && plan.n_leaves <= 64 && rows_fast_ok(x, g, q, n))
        return launch_rows_prologue<PRO_RMSNORM>(s, x, g, rows, n, eps, plan, q, scales, nullptr, 0, packed, pf);
    if (packed) return hipErrorInvalidValue;
    const size_t lds = sizeof(float) * ((size_t)2 * n + 10 * (size_t)plan.n_leaves + 16);
    TL_KLAUNCH(rmsnorm_quant_kernel, dim3(rows), dim3(256), lds, s, x, g, n, eps, plan, y, q, scales);
    return hipGetLastError();
}

hipError_t launch_quantize_rows(hipStream_t s, const float* x, int32_t rows, int32_t n, int8_t* q,
                                double* scales, int32_t* zero, int32_t zero_n, bool packed, const L2Prefetch* pf) {
    if (rows <= 0) return hipSuccess;
    if ((zero || packed) && !rows_fast_ok(x, nullptr, q, n)) return hipErrorInvalidValue;
    if (zero && (zero_n <= 0 || zero_n % 4 || (uintptr_t)zero % 16)) return hipErrorInvalidValue;
    if (rows_fast_ok(x, nullptr, q, n))
        return launch_rows_prologue<PRO_QUANT>(s, x, nullptr, rows, n, 0.0f, PwPlan{8, 1}, q, scales, zero, zero_n,
                                               packed, pf);
    TL_KLAUNCH(quantize_rows_kernel<false>, dim3(rows), dim3(256), 0, s, x, n, q, (void*)scales);
    return hipGetLastError();
}

hipError_t launch_quantize_weight_rows(hipStream_t s, const float* w, int32_t rows, int32_t n,
                                       int8_t* q, float* scales) {
    if (rows <= 0) return hipSuccess;
    TL_KLAUNCH(quantize_rows_kernel<true>, dim3(rows), dim3(256), 0, s, w, n, q, (void*)scales);
    return hipGetLastError();
}

hipError_t launch_quantize_tensor(hipStream_t s, const float* x, int64_t n, int8_t* q,
                                  double* scale, float* scratch_max) {
    unsigned* mx = (unsigned*)scratch_max;
    TL_KLAUNCH(fill_u32_kernel, dim3(1), dim3(64), 0, s, mx, 1, 0u);
    const int blocks = (int)std::min<int64_t>(1024, std::max<int64_t>(1, (n + 255) / 256));
    if (n > 0) TL_KLAUNCH(tensor_absmax_kernel, dim3(blocks), dim3(256), 0, s, x, n, mx);
    TL_KLAUNCH(tensor_quant_kernel, dim3(blocks), dim3(256), 0, s, x, n, mx, q, scale);
    return hipGetLastError();
}

template <int R, int EPI>
static hipError_t gemv_r(hipStream_t s, const GemvArgs& a) {
    const int kch = ceil_div(a.k, 1024);
    const dim3 grid(ceil_div(a.n, 4 * R)), block(256);
    switch (kch) {
        case 1: TL_KLAUNCH((gemv_kernel<R, 1, EPI>), grid, block, 0, s, a); break;
        case 2: TL_KLAUNCH((gemv_kernel<R, 2, EPI>), grid, block, 0, s, a); break;
        case 3: TL_KLAUNCH((gemv_kernel<R, 3, EPI>), grid, block, 0, s, a); break;
        case 4: TL_KLAUNCH((gemv_kernel<R, 4, EPI>), grid, block, 0, s, a); break;
        case 5: TL_KLAUNCH((gemv_kernel<R, 5, EPI>), grid, block, 0, s, a); break;
        case 6: TL_KLAUNCH((gemv_kernel<R, 6, EPI>), grid, block, 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int EPI>
static hipError_t gemv_epi(hipStream_t s, const GemvArgs& a) {
    // rows per wavefront: enough workgroups to cover the chip, enough bytes in
    // flight per lane
    const int kch = ceil_div(a.k, 1024);
    if (EPI == EPI_GLU || kch > 3) return gemv_r<2, EPI>(s, a);
    if (a.n >= 8192) return gemv_r<4, EPI>(s, a);
    return gemv_r<2, EPI>(s, a);
}

hipError_t launch_gemv(hipStream_t s, int epi, const GemvArgs& a) {
    if (a.n <= 0) return hipSuccess;
    if (a.k <= 0 || a.k % 16 != 0 || a.k > 6 * 1024) return hipErrorInvalidValue;
    switch (epi) {
        case EPI_DEQUANT: return gemv_epi<EPI_DEQUANT>(s, a);
        case EPI_DEQUANT_RES: return gemv_epi<EPI_DEQUANT_RES>(s, a);
        case EPI_REQUANT: return gemv_epi<EPI_REQUANT>(s, a);
        case EPI_GLU: return gemv_epi<EPI_GLU>(s, a);
        case EPI_ARGMAX: return gemv_epi<EPI_ARGMAX>(s, a);
        case EPI_RAW: return gemv_epi<EPI_REQUANT>(s, a);  // y8 unused when only acc wanted
        default: return hipErrorInvalidValue;
    }
}

template <int WTM, int WTN, int EPI>
static void gemm_go(hipStream_t s, const GemmArgs& a, int32_t splits) {
    constexpr int BM = 32 * WTM, BN = 32 * WTN;
    const dim3 grid(ceil_div(a.n, BN), ceil_div(a.m, BM), splits);
    TL_KLAUNCH((gemm_kernel<WTM, WTN, EPI>), grid, dim3(256), 0, s, a);
}

template <int EPI>
static void gemm_shape(hipStream_t s, const GemmArgs& a, int32_t splits) {
    if (a.m <= 32) gemm_go<1, 2, EPI>(s, a, splits);
    else gemm_go<2, 2, EPI>(s, a, splits);
}

hipError_t launch_gemm(hipStream_t s, int epi, const GemmArgs& a, int32_t splits) {
    if (a.m <= 0 || a.n <= 0) return hipSuccess;
    if (a.k <= 0 || a.k % 64 != 0 || a.k_split % 64 != 0 || splits < 1) return hipErrorInvalidValue;
    switch (epi) {
        case EPI_DEQUANT: gemm_shape<EPI_DEQUANT>(s, a, splits); break;
        case EPI_DEQUANT_RES: gemm_shape<EPI_DEQUANT_RES>(s, a, splits); break;
        case EPI_GLU: gemm_shape<EPI_GLU>(s, a, splits); break;
        case EPI_RAW: gemm_shape<EPI_RAW>(s, a, splits); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// small-M GEMM without a cross-workgroup reduction: one workgroup of 16
// wavefronts per 32-column output tile; wavefront w multiplies the 32 A rows
// by the tile's weight rows over its own run of consecutive 32-byte K chunks
// (register loads, all issued before the first MFMA) and the 16 partial
// tiles are added in LDS (exact integers) by the epilogue threads, one
// output element each.  Used for K <= 2048; the split-K kernel covers the
// long-K down projection with more workgroups.
constexpr int kRowsWaves = 16;
constexpr int kRowsChunks = 12;   // most 32-byte K chunks per wavefront (K <= 16 x 12 x 32 = 6144)

// PK: the weights are read from their packed copy (a.wp / a.wp2, MFMA
// operand order, one contiguous 1 KiB block per 32 rows x 32 K bytes), so
// every weight load of a wavefront is one coalesced 1 KiB read; otherwise from
// the row-major [N][K] matrix (32 rows x 32 bytes per load).
//
// K slices (EPI_ACC): blockIdx.y takes the 32-byte chunks
// [y (k_split / 32), (y + 1) (k_split / 32)) of K, and the slice's integer
// sums are added into acc with device-scope atomics (exact: the order of
// integer additions does not change the sum)
template <int EPI, int CH, bool PK, int W = kRowsWaves>
__global__ __launch_bounds__(W * 64) void gemm_rows32_kernel(GemmArgs a) {
    constexpr int NB = EPI == EPI_GLU ? 2 : 1;
    extern __shared__ __align__(16) int rows32_lds[];   // [W waves][NB][16][64]
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id(), col = lane & 31, hi = lane >> 5;
    const int n0 = blockIdx.x * 32;
    const int cps = a.k_split >> 5, c0 = blockIdx.y * cps;
    const int kch = min(cps, (a.k >> 5) - c0);   // chunks of this K slice (>= 1)
    const int8_t* arow = a.a + (int64_t)min(col, a.m - 1) * a.k + (int64_t)c0 * 32 + hi * 16;
    const int8_t* wrow[NB];
    if (PK) {
        const int64_t o = ((int64_t)blockIdx.x * (a.k >> 5) + c0) * 1024 + lane * 16;
        wrow[0] = a.wp + o;
        if (NB == 2) wrow[NB - 1] = a.wp2 + o;
    } else {
        const int64_t o = (int64_t)min(n0 + col, a.n - 1) * a.k + (int64_t)c0 * 32 + hi * 16;
        wrow[0] = a.w + o;
        if (NB == 2) wrow[NB - 1] = a.w2 + o;
    }
    const int64_t wstep = PK ? 1024 : 32;   // bytes between consecutive K chunks
    const int per = (kch + W - 1) / W;   // consecutive chunks of this wavefront: 4 loads cover a 128-byte line
    // the epilogue's operands of this wavefront's output elements (registers
    // i = wave + W ii of every lane: row 8 (i / 4) + 4 (l / 32) + i % 4,
    // column n0 + l % 32) are requested first, so they arrive with the first
    // weight loads instead of after the LDS fold (indices clamped in range;
    // out-of-range elements are not stored)
    constexpr int NI = 16 / W;
    double esx[NI];
    float eres[NI], esw = 0.0f, esw2 = 0.0f;
    if constexpr (EPI != EPI_RAW && EPI != EPI_ACC && EPI != EPI_ACC_F32) {
        const int en = min(n0 + col, a.n - 1);
        esw = a.ws[en];
        if constexpr (EPI == EPI_GLU) esw2 = a.ws2[en];
#pragma unroll
        for (int ii = 0; ii < NI; ii++) {
            const int i = wave + W * ii, mc = min(8 * (i >> 2) + 4 * hi + (i & 3), a.m - 1);
            esx[ii] = a.as[mc];
            if constexpr (EPI == EPI_DEQUANT_RES) eres[ii] = a.residual[(int64_t)mc * a.n + en];
        }
    }
    v4i af[CH], bf[NB][CH];
    if constexpr (EPI == EPI_ACC_F32) {
        // a float32 A (a.af; one 32-byte K chunk per wavefront,
        // which the launcher checks): this lane's 16 values of its row are
        // requested first, then the weights, then quantized as
        // quantize_rows_kernel does, at the row maximum
        const int rq = min(col, a.m - 1), cc = min(wave * per, kch - 1);
        // the row's amax_n maxima: float4 2 q + hi of this lane (clamped;
        // max is idempotent), the other half-wavefront's in the lane l ^ 32
        const float4* m4 = (const float4*)(a.amax + (int64_t)rq * a.amax_n);
        float4 mv[4];
#pragma unroll
        for (int q = 0; q < 4; q++) mv[q] = m4[min(2 * q + hi, (a.amax_n >> 2) - 1)];
        const float4* f4 = (const float4*)(a.af + (int64_t)rq * a.k + (int64_t)(c0 + cc) * 32 + hi * 16);
        float4 fv[4];
#pragma unroll
        for (int w = 0; w < 4; w++) fv[w] = f4[w];
        float mx = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; q++) mx = fmaxf(fmaxf(fmaxf(mx, mv[q].x), fmaxf(mv[q].y, mv[q].z)), mv[q].w);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
#pragma unroll
        for (int j = 0; j < CH; j++) {
            const int ccj = min(wave * per + min(j, per - 1), kch - 1);
#pragma unroll
            for (int b = 0; b < NB; b++) bf[b][j] = ld_nt16(wrow[b] + (int64_t)ccj * wstep);
        }
        const double s = quant_scale(mx);
        if (blockIdx.x == 0 && blockIdx.y == 0 && wave == 0 && hi == 0 && col < a.m) a.as_out[col] = s;
        RnDiv dv;
        dv.b = (float)s;
        dv.y = __fdiv_rn(1.0f, dv.b);
        dv.fast = __all(fabsf(dv.b) >= 0x1p-64f && fabsf(dv.b) <= 0x1p64f);
        // |x| <= max |x| = 127 b (1 + 2^-24) keeps every x y finite
#pragma unroll
        for (int w = 0; w < 4; w++) af[0][w] = (int)(dv.fast ? quant4<true>(fv[w], dv) : quant4<false>(fv[w], dv));
#pragma unroll
        for (int j = 1; j < CH; j++) af[j] = (v4i){0, 0, 0, 0};   // unused (one chunk)
    } else {
#pragma unroll
        for (int j = 0; j < CH; j++) {
            const int cc = min(wave * per + min(j, per - 1), kch - 1);
            af[j] = ld16(arow + (int64_t)cc * 32);
#pragma unroll
            for (int b = 0; b < NB; b++) bf[b][j] = ld_nt16(wrow[b] + (int64_t)cc * wstep);
        }
    }
    v16i acc[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) acc[b] = (v16i){};
#pragma unroll
    for (int j = 0; j < CH; j++)
        if (j < per && wave * per + j < kch)
#pragma unroll
            for (int b = 0; b < NB; b++) acc[b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[j], bf[b][j], acc[b], 0, 0, 0);
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int i = 0; i < 16; i++) rows32_lds[((wave * NB + b) * 16 + i) * 64 + lane] = acc[b][i];
    __syncthreads();
    // the tile's 16 x 64 (register i, lane l) elements: wavefront w finishes
    // registers w, w + W, ... of every lane
    const int l = lane;
#pragma unroll
    for (int ii = 0; ii < NI; ii++) {
        const int i = wave + W * ii;
        const int m = 8 * (i >> 2) + 4 * (l >> 5) + (i & 3), n = n0 + (l & 31);
        if (EPI == EPI_ARGMAX) {
            // dequantized logit -> 64-bit key; the 32 columns of row m are the
            // 32 lanes of this half-wavefront, whose best key is this tile's key
            // of row m (argmax_tiles_kernel folds the tiles)
            unsigned long long k = 0;
            if (m < a.m && n < a.n) {
                int v = 0;
#pragma unroll
                for (int w = 0; w < W; w++) v += rows32_lds[(w * 16 + i) * 64 + l];
                const float lg = (float)v * deq_mult(esx[ii], esw);
                if (a.y) a.y[(int64_t)m * a.n + n] = lg;
                k = argmax_key(lg, n);
            }
            k = half_max_u64(k);
            if ((l & 31) == 0 && m < a.m) a.key[(int64_t)blockIdx.x * a.m + m] = k;
            continue;
        }
        if (m >= a.m || n >= a.n) continue;
        int sum[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            int v = 0;
#pragma unroll
            for (int w = 0; w < W; w++) v += rows32_lds[((w * NB + b) * 16 + i) * 64 + l];
            sum[b] = v;
        }
        const int64_t idx = (int64_t)m * a.n + n;
        if (EPI == EPI_RAW) {
            a.acc[idx] = sum[0];
        } else if (EPI == EPI_ACC || EPI == EPI_ACC_F32) {
            __hip_atomic_fetch_add(a.acc + idx, sum[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            const double sx = esx[ii];
            const float v0 = (float)sum[0] * deq_mult(sx, esw);
            if (EPI == EPI_GLU) {
                const float up = (float)sum[NB - 1] * deq_mult(sx, esw2);
                a.y[idx] = tl_silu(v0) * up;
            } else if (EPI == EPI_DEQUANT_RES) {
                a.y[idx] = eres[ii] + v0;
            } else {
                a.y[idx] = v0;
            }
        }
    }
}

static size_t rows32_lds_bytes(int nb, int w = kRowsWaves) { return (size_t)w * nb * 16 * 64 * sizeof(int); }

// the 8-wavefront variant on packed weights (gate/up: with 8 its GEMM took
// 225 against 273 us per batched step at 32 x 2048): 8 chunks of 32 bytes per
// wavefront, so a K slice of at most 2048 bytes
template <int W>
static hipError_t launch_rows32_w(hipStream_t s, int epi, const GemmArgs& a, dim3 grid) {
    constexpr int CH = 64 / W;
    const dim3 block(W * 64);
    const size_t lds1 = rows32_lds_bytes(1, W), lds2 = rows32_lds_bytes(2, W);
    switch (epi) {
        case EPI_DEQUANT: TL_KLAUNCH((gemm_rows32_kernel<EPI_DEQUANT, CH, true, W>), grid, block, lds1, s, a); break;
        case EPI_DEQUANT_RES: TL_KLAUNCH((gemm_rows32_kernel<EPI_DEQUANT_RES, CH, true, W>), grid, block, lds1, s, a); break;
        case EPI_GLU: TL_KLAUNCH((gemm_rows32_kernel<EPI_GLU, CH, true, W>), grid, block, lds2, s, a); break;
        case EPI_RAW: TL_KLAUNCH((gemm_rows32_kernel<EPI_RAW, CH, true, W>), grid, block, lds1, s, a); break;
        case EPI_ACC: TL_KLAUNCH((gemm_rows32_kernel<EPI_ACC, CH, true, W>), grid, block, lds1, s, a); break;
        case EPI_ARGMAX: TL_KLAUNCH((gemm_rows32_kernel<EPI_ARGMAX, CH, true, W>), grid, block, lds1, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// M <= 32, K a multiple of 64 and at most 6144; with packed weights (a.wp,
// and a.wp2 for the GLU) N must be a multiple of 32.  a.k_split (a multiple
// of 32, 0 = K) slices K over gridDim.y workgroups for EPI_ACC.  waves = 8
// runs 8-wavefront workgroups (packed weights, K slice at most 2048 bytes),
// else 16.
hipError_t launch_gemm_rows32(hipStream_t s, int epi, const GemmArgs& args, int32_t waves) {
    GemmArgs a = args;
    if (a.m < 1 || a.m > 32 || a.n <= 0 || a.k <= 0 || a.k % 64 || a.k > kRowsWaves * kRowsChunks * 32)
        return hipErrorInvalidValue;
    if (a.k_split <= 0 || a.k_split >= a.k || (epi != EPI_ACC && epi != EPI_ACC_F32)) a.k_split = a.k;
    if (a.k_split % 32) return hipErrorInvalidValue;
    if ((epi == EPI_ACC || epi == EPI_ACC_F32) && !a.acc) return hipErrorInvalidValue;
    if (epi == EPI_ARGMAX && !a.key) return hipErrorInvalidValue;
    const bool pk = a.wp != nullptr;
    if (pk && (a.n % 32 || (epi == EPI_GLU && !a.wp2))) return hipErrorInvalidValue;
    // a float32 A (quantized in the kernel): the 16-wavefront kernel with one
    // 32-byte K chunk per wavefront, 16-byte aligned rows
    if (epi == EPI_ACC_F32 && (!pk || !a.af || !a.a || !a.amax || a.amax_n < 4 || a.amax_n > 32 || a.amax_n % 4 ||
                                   (uintptr_t)a.amax % 16 || !a.as_out || a.k_split / 32 > kRowsWaves ||
                 a.k % 4 || (uintptr_t)a.af % 16))
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)((a.n + 31) / 32), (unsigned)((a.k + a.k_split - 1) / a.k_split));
    if (pk && waves == 8 && a.k_split <= 64 * 32 && epi != EPI_ACC_F32) return launch_rows32_w<8>(s, epi, a, grid);
    const dim3 block(1024);
    const size_t lds1 = rows32_lds_bytes(1), lds2 = rows32_lds_bytes(2);
    const bool shortk = a.k_split <= kRowsWaves * 4 * 32;
#define TL_R32P(E, C, L)                                                                    \
    do {                                                                                    \
        if (pk) TL_KLAUNCH((gemm_rows32_kernel<E, C, true>), grid, block, L, s, a);         \
        else TL_KLAUNCH((gemm_rows32_kernel<E, C, false>), grid, block, L, s, a);           \
    } while (0)
#define TL_R32(E, L)                                                                        \
    do {                                                                                    \
        if (shortk) TL_R32P(E, 4, L);                                                       \
        else TL_R32P(E, kRowsChunks, L);                                                    \
    } while (0)
    switch (epi) {
        case EPI_DEQUANT: TL_R32(EPI_DEQUANT, lds1); break;
        case EPI_DEQUANT_RES: TL_R32(EPI_DEQUANT_RES, lds1); break;
        case EPI_GLU:
            if (!shortk) return hipErrorInvalidValue;   // both weight sets of 12 chunks exceed the registers
            TL_R32P(EPI_GLU, 4, lds2);
            break;
        case EPI_RAW: TL_R32(EPI_RAW, lds1); break;
        case EPI_ACC: TL_R32(EPI_ACC, lds1); break;
        case EPI_ACC_F32: TL_KLAUNCH((gemm_rows32_kernel<EPI_ACC_F32, 4, true>), grid, block, lds1, s, a); break;
        case EPI_ARGMAX:
            if (!shortk) return hipErrorInvalidValue;
            TL_R32P(EPI_ARGMAX, 4, lds1);
            break;
        default: return hipErrorInvalidValue;
    }
#undef TL_R32
#undef TL_R32P
    return hipGetLastError();
}

// packed copy of an int8 [N][K] matrix (N, K multiples of 32): block
// (n / 32, k / 32) of 1 KiB at ((n / 32) (K / 32) + k / 32) * 1024, byte
// (((k / 16) % 2) * 32 + n % 32) * 16 + k % 16 -- lane l of an MFMA B operand
// (row l % 32, K bytes 16 (l / 32) .. +16) reads bytes 16 l .. 16 l + 15
__global__ __launch_bounds__(256) void pack_weights_kernel(const int8_t* __restrict__ w, int32_t n, int32_t k,
                                                           int8_t* __restrict__ wp) {
    const int64_t units = (int64_t)n * k / 16;
    const int kch = k >> 5;
    for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units; u += (int64_t)gridDim.x * blockDim.x) {
        const int64_t blk = u >> 6;
        const int l = (int)(u & 63);
        const int64_t nb = blk / kch, kc = blk % kch;
        const int8_t* src = w + (nb * 32 + (l & 31)) * (int64_t)k + kc * 32 + (l >> 5) * 16;
        *(v4i*)(wp + u * 16) = *(const v4i*)src;
    }
}

hipError_t launch_pack_weights(hipStream_t s, const int8_t* w, int32_t n, int32_t k, int8_t* wp) {
    if (n <= 0 || k <= 0 || n % 32 || k % 32) return hipErrorInvalidValue;
    const int64_t units = (int64_t)n * k / 16;
    const int blocks = (int)std::min<int64_t>(8192, (units + 255) / 256);
    TL_KLAUNCH(pack_weights_kernel, dim3(blocks), dim3(256), 0, s, w, n, k, wp);
    return hipGetLastError();
}

// staging of 4 wavefronts (A + NB weight tiles of 32 x 256 bytes); also
// holds the wavefront partials and the other slices' tiles (8 x NB x 4 KiB)
static size_t skinny_lds_bytes(int nb) { return (size_t)4 * (1 + nb) * 8192; }

hipError_t init_skinny_kernels() {
    hipError_t e = hipSuccess;
    const void* fns[4] = {(const void*)gemm_skinny_kernel<EPI_DEQUANT>, (const void*)gemm_skinny_kernel<EPI_DEQUANT_RES>,
                          (const void*)gemm_skinny_kernel<EPI_GLU>, (const void*)gemm_skinny_kernel<EPI_RAW>};
    for (int i = 0; i < 4 && e == hipSuccess; i++)
        e = hipFuncSetAttribute(fns[i], hipFuncAttributeMaxDynamicSharedMemorySize, (int)skinny_lds_bytes(i == 2 ? 2 : 1));
#define TL_R32FNS(PK)                                                                                    \
    {(const void*)gemm_rows32_kernel<EPI_DEQUANT, 4, PK>, (const void*)gemm_rows32_kernel<EPI_DEQUANT_RES, 4, PK>, \
     (const void*)gemm_rows32_kernel<EPI_RAW, 4, PK>, (const void*)gemm_rows32_kernel<EPI_DEQUANT, kRowsChunks, PK>, \
     (const void*)gemm_rows32_kernel<EPI_DEQUANT_RES, kRowsChunks, PK>,                                  \
     (const void*)gemm_rows32_kernel<EPI_RAW, kRowsChunks, PK>, (const void*)gemm_rows32_kernel<EPI_GLU, 4, PK>, \
     (const void*)gemm_rows32_kernel<EPI_ARGMAX, 4, PK>}
    const void* rfns[2][8] = {TL_R32FNS(false), TL_R32FNS(true)};
#undef TL_R32FNS
    for (int p = 0; p < 2; p++)
        for (int i = 0; i < 8 && e == hipSuccess; i++)
            e = hipFuncSetAttribute(rfns[p][i], hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)rows32_lds_bytes(i == 6 ? 2 : 1));
    return e;
}

// M <= 32, K a multiple of 64; `part` holds tiles x slices x NB x 1024
// int32 when slices > 1, `counters` one zeroed word per output tile
hipError_t launch_gemm_skinny(hipStream_t s, int epi, const GemmArgs& a, int32_t slices, int32_t* part,
                              unsigned* counters) {
    if (a.m < 1 || a.m > 32 || a.n <= 0 || a.k <= 0 || a.k % 64 || slices < 1 || slices > kSkinnyMaxSlices)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)(((a.n + 31) / 32) * slices)), block(256);
    const size_t lds1 = skinny_lds_bytes(1), lds2 = skinny_lds_bytes(2);
    switch (epi) {
        case EPI_DEQUANT: TL_KLAUNCH(gemm_skinny_kernel<EPI_DEQUANT>, grid, block, lds1, s, a, slices, part, counters); break;
        case EPI_DEQUANT_RES: TL_KLAUNCH(gemm_skinny_kernel<EPI_DEQUANT_RES>, grid, block, lds1, s, a, slices, part, counters); break;
        case EPI_GLU: TL_KLAUNCH(gemm_skinny_kernel<EPI_GLU>, grid, block, lds2, s, a, slices, part, counters); break;
        case EPI_RAW: TL_KLAUNCH(gemm_skinny_kernel<EPI_RAW>, grid, block, lds1, s, a, slices, part, counters); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemm_reduce(hipStream_t s, int epi, const GemmArgs& a, int32_t splits) {
    const int blocks = (int)std::min<int64_t>(2048, ((int64_t)a.m * a.n + 255) / 256);
    switch (epi) {
        case EPI_DEQUANT: TL_KLAUNCH(gemm_reduce_kernel<EPI_DEQUANT>, dim3(blocks), dim3(256), 0, s, a, splits); break;
        case EPI_DEQUANT_RES: TL_KLAUNCH(gemm_reduce_kernel<EPI_DEQUANT_RES>, dim3(blocks), dim3(256), 0, s, a, splits); break;
        case EPI_GLU: TL_KLAUNCH(gemm_reduce_kernel<EPI_GLU>, dim3(blocks), dim3(256), 0, s, a, splits); break;
        case EPI_RAW: TL_KLAUNCH(gemm_reduce_kernel<EPI_RAW>, dim3(blocks), dim3(256), 0, s, a, splits); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_qkv_post(hipStream_t s, const float* qkv, int32_t rows, int32_t n_heads,
                           int32_t n_kv_heads, RowMap rm, const float* cos, const float* sin,
                           KvGeom kv, int32_t layer, const float* kv_sk, const float* kv_sv,
                           int8_t* q8, double* q_scale, float* q_rot_out, bool append_kv) {
    if (rows <= 0) return hipSuccess;
    const int D = n_heads * kHeadDim, KVD = n_kv_heads * kHeadDim;
    const size_t lds = sizeof(float) * ((size_t)(D + 2 * KVD) + D + KVD);
    TL_KLAUNCH(qkv_post_kernel, dim3(rows), dim3(256), lds, s, qkv, n_heads, n_kv_heads, rm,
                       cos, sin, kv, layer, kv_sk, kv_sv, q8, q_scale, q_rot_out, (int32_t)append_kv);
    return hipGetLastError();
}

// INT8 probabilities of 32 rows x tpad keys, block sums, partial sums
static size_t tile_lds_bytes(int tpad) { return (size_t)32 * tpad + (size_t)32 * (tpad / 64) * sizeof(float) + 32 * 64 * sizeof(int); }

hipError_t init_prefill_kernels() {
    return hipFuncSetAttribute((const void*)attention_tile_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)tile_lds_bytes(kTileMaxKeys));
}

// the same computation for contexts of at most 128 NB keys per wavefront
// (NB blocks of 64 each, i.e. tpad <= 256 NB), in the transposed layout
// S^T = K Q^T: lane l owns query row l % 32 and register i key
// 8 (i / 4) + 4 (l / 32) + i % 4 of a 32-key tile.  A row's maximum is then
// an in-lane maximum and one exchange with lane l ^ 32; of the block-64
// butterfly (token distances 32, 16, 8, 4, 2, 1) only distance 4 (lane
// l ^ 32) crosses lanes, the others add registers of one lane; four
// probabilities of a lane are consecutive keys and leave as one 32-bit LDS
// store.  Every K and V fragment of the wavefront is requested at the start;
// scores and exponentials stay in registers across the passes.
template <int NB>
__global__ __launch_bounds__(256) void attention_tile_reg_kernel(AttnTileArgs p) {
    extern __shared__ __align__(16) int8_t tile_lds[];
    __shared__ __align__(16) int8_t qs8[32 * 64];   // Q quantized by the workgroup (float32 Q input)
    __shared__ float scl[32], tot[32];
    __shared__ float wmax[4][32];
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int col = lane & 31, hi = lane >> 5;
    const int h = blockIdx.x, r0 = (gridDim.y - 1 - blockIdx.y) * 32;   // the longest (last) tiles dispatch first
    const int G = p.n_heads / p.n_kv, g = h / G;
    const int nr = min(32, p.rows - r0);
    const int pos_first = p.pos0 + r0;
    const int T = pos_first + nr;
    const int tpad = (T + 63) & ~63, nblk = tpad >> 6;
    int8_t* p8 = tile_lds;                         // [32][tpad]
    float* bsum = (float*)(tile_lds + 32 * tpad);  // [32][nblk]
    int* accs = (int*)(bsum + 32 * nblk);          // [32][64]
    const int D = p.n_heads * kHeadDim;
    const int64_t pl = p.kv.plane(p.seq, p.layer, g);
    const int8_t* kp = p.kv.k + pl;
    const int8_t* vp = p.kv.v + pl;
    const float sk = p.kv_sk[p.layer * p.n_kv + g], sv = p.kv_sv[p.layer * p.n_kv + g];

    // every load first: Q, then K of this wavefront's blocks b = wave + 4 j
    // (two 32-key tiles each), then V of its 32-key chunks c = wave + 4 j.
    // Blocks and chunks past the tile's keys (b >= nblk, c >= tpad / 32: a
    // short causal tile) are skipped here and in every pass below -- each
    // test is uniform per wavefront -- so a short tile costs less than the
    // longest instead of the same.
    TileQ tq;
    tile_q_load(p, r0, nr, h, col, hi, tq);
    v4i kf[NB][2][2], vf[2 * NB][2];
#pragma unroll
    for (int j = 0; j < NB; j++) {
        if (wave + 4 * j >= nblk) continue;
#pragma unroll
        for (int half = 0; half < 2; half++) {
            const int t = 64 * (wave + 4 * j) + 32 * half + col;
            const int8_t* kb = kp + (int64_t)(t >> 6) * 4096 + hi * 1024 + (t & 63) * 16;
            kf[j][half][0] = ld16(kb);
            kf[j][half][1] = ld16(kb + 2048);
        }
    }
#pragma unroll
    for (int j = 0; j < 2 * NB; j++) {
        const int kc = wave + 4 * j;
        if (kc >= tpad / 32) continue;
        const int8_t* vb = vp + (int64_t)(kc * 2 + hi) * 1024 + col * 16;
        vf[j][0] = ld16(vb);
        vf[j][1] = ld16(vb + 512);
    }
    if (tid < 32) scl[tid] = (float)((tile_q_scale(p, r0 + min(tid, nr - 1)) * (double)sk) * p.attn_scale);
    for (int e = tid; e < 32 * 64; e += 256) accs[e] = 0;
    tile_q_quantize(p, tq, qs8);   // float32 Q quantized while the K and V loads are in flight
    __syncthreads();
    tile_q_frags(p, qs8, col, hi, tq);
    const v4i qa0 = tq.qa0, qa1 = tq.qa1;
    const float rs = scl[col];
    const int rpos = pos_first + col;

    // pass A: scores (kept) and the row maximum
    float sc[NB][2][16];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NB; j++) {
        if (wave + 4 * j >= nblk) continue;
#pragma unroll
        for (int half = 0; half < 2; half++) {
            v16i acc = {};
            acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf[j][half][0], qa0, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf[j][half][1], qa1, acc, 0, 0, 0);
            const int t0 = 64 * (wave + 4 * j) + 32 * half + 4 * hi;
            if (64 * (wave + 4 * j) + 63 <= pos_first) {   // every row sees the whole block
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float v = (float)acc[i] * rs;
                    sc[j][half][i] = v;
                    mx = fmaxf(mx, v);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float v = (float)acc[i] * rs;
                    sc[j][half][i] = v;
                    const int t = t0 + 8 * (i >> 2) + (i & 3);
                    mx = t <= rpos ? fmaxf(mx, v) : mx;
                }
            }
        }
    }
    mx = fmaxf(mx, lane_xor<32>(mx));
    if (hi == 0) wmax[wave][col] = mx;
    __syncthreads();
    const float m = fmaxf(fmaxf(wmax[0][col], wmax[1][col]), fmaxf(wmax[2][col], wmax[3][col]));

    // pass B: exponentials (kept) and block sums in the butterfly order
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const int b = wave + 4 * j;
        if (b >= nblk) continue;
        const int t0 = 64 * b + 4 * hi;
        // x - m <= 0 for every key a row sees: tl_expf_nonpos is tl_expf there
        if (64 * b + 63 <= pos_first) {
#pragma unroll
            for (int half = 0; half < 2; half++)
#pragma unroll
                for (int i = 0; i < 16; i++) sc[j][half][i] = tl_expf_nonpos(sc[j][half][i] - m);
        } else {
#pragma unroll
            for (int half = 0; half < 2; half++)
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int t = t0 + 32 * half + 8 * (i >> 2) + (i & 3);
                    sc[j][half][i] = t <= rpos ? tl_expf_nonpos(sc[j][half][i] - m) : 0.0f;
                }
        }
        float a[16];
#pragma unroll
        for (int i = 0; i < 16; i++) a[i] = sc[j][0][i] + sc[j][1][i];      // distance 32
        float c[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float b0 = a[r] + a[r + 8], b1 = a[r + 4] + a[r + 12];      // distance 16
            c[r] = b0 + b1;                                                   // distance 8
        }
        float d[4];
#pragma unroll
        for (int r = 0; r < 4; r++) d[r] = pair_sum<32>(c[r]);      // distance 4
        const float f = (d[0] + d[2]) + (d[1] + d[3]);                        // distances 2, 1
        if (hi == 0) bsum[col * nblk + b] = f;
    }
    __syncthreads();
    if (tid < 32) {
        const float total = ordered_sum(bsum + tid * nblk, nblk);
        tot[tid] = total;
    }
    __syncthreads();

    // pass C: INT8 probabilities, four consecutive keys per 32-bit store;
    // exponential / total correctly rounded from the row's reciprocal and two
    // residual corrections (e <= 1 <= total keeps e y finite; the wave vote
    // confirms every total lies in the quotient's range).  A float sum of
    // nonnegative terms is never below any of them, so 0 <= e <= total and
    // rne(127 e / total) already lies in [0, 127]: the probability clip holds
    // without a clamp, and the byte is packed straight from the float.
    const float tr = tot[col];
    const RnDiv dv{tr, __fdiv_rn(1.0f, tr), true};
    const bool fast = __all(fabsf(tr) >= 0x1p-64f && fabsf(tr) <= 0x1p64f);
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const int b = wave + 4 * j;
        if (b < nblk) {
#pragma unroll
            for (int half = 0; half < 2; half++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    unsigned word = 0;
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float e = sc[j][half][4 * q + r];
                        const float pr = __builtin_rintf((fast ? rn_div_fast(e, dv) : __fdiv_rn(e, tr)) * 127.0f);
                        word = __builtin_amdgcn_cvt_pk_u8_f32(pr, r, word);
                    }
                    *(unsigned*)(p8 + col * tpad + 64 * b + 32 * half + 8 * q + 4 * hi) = word;
                }
        }
    }
    __syncthreads();

    // pass D: O = P8 . V
    v16i o0 = {}, o1 = {};
#pragma unroll
    for (int j = 0; j < 2 * NB; j++) {
        const int kc = wave + 4 * j;
        if (kc < tpad / 32) {
            const v4i a = *(const v4i*)(p8 + col * tpad + kc * 32 + hi * 16);
            o0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, vf[j][0], o0, 0, 0, 0);
            o1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, vf[j][1], o1, 0, 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int r = 8 * (i >> 2) + 4 * hi + (i & 3);
        atomicAdd(&accs[r * 64 + col], o0[i]);
        atomicAdd(&accs[r * 64 + 32 + col], o1[i]);
    }
    __syncthreads();
    const float pv_mult = deq_mult(1.0 / 127.0, sv);
    for (int e = tid; e < 32 * 64; e += 256) {
        const int r = e >> 6, d = e & 63;
        if (r < nr) p.out[(int64_t)(r0 + r) * D + (int64_t)h * kHeadDim + d] = (float)accs[e] * pv_mult;
    }
}

// rows of one sequence at positions pos0 .. pos0 + rows - 1
hipError_t launch_attention_tiles(hipStream_t s, const int8_t* q8, const double* q_scale, int32_t rows,
                                  int32_t n_heads, int32_t n_kv_heads, int32_t seq, int32_t pos0, KvGeom kv,
                                  int32_t layer, const float* kv_sk, const float* kv_sv, float* out,
                                  const float* qf, const unsigned* qmax) {
    if (rows <= 0) return hipSuccess;
    if (n_heads % n_kv_heads || pos0 < 0 || pos0 + rows > kv.max_pos || pos0 + rows > kTileMaxKeys ||
        (qf && !qmax) || (!qf && (!q8 || !q_scale)))
        return hipErrorInvalidValue;
    const int tpad = (pos0 + rows + 63) & ~63;
    const size_t lds = tile_lds_bytes(tpad);
    AttnTileArgs a{q8, q_scale, n_heads, n_kv_heads, rows, seq, pos0, layer, kv, kv_sk, kv_sv,
                   1.0 / sqrt((double)kHeadDim), out, qf, qmax};
    const dim3 grid(n_heads, (rows + 31) / 32), block(256);
    if (tpad <= 256) TL_KLAUNCH(attention_tile_reg_kernel<1>, grid, block, lds, s, a);
    else if (tpad <= 512) TL_KLAUNCH(attention_tile_reg_kernel<2>, grid, block, lds, s, a);
    else TL_KLAUNCH(attention_tile_kernel, grid, block, lds, s, a);
    return hipGetLastError();
}

hipError_t launch_attention(hipStream_t s, const int8_t* q8, const double* q_scale, int32_t rows,
                            int32_t n_heads, int32_t n_kv_heads, RowMap rm, KvGeom kv,
                            int32_t layer, const float* kv_sk, const float* kv_sv, float* out,
                            int32_t max_t, AttnDebug dbg) {
    if (rows <= 0) return hipSuccess;
    const int G = n_heads / n_kv_heads;
    if (G < 1 || G > kMaxGroup || n_heads % n_kv_heads) return hipErrorInvalidValue;
    const int tpad = (max_t + 63) & ~63;
    const size_t lds = (size_t)G * tpad * sizeof(float) + (size_t)G * tpad + (size_t)G * (tpad / 64) * sizeof(float) + 16;
    const double attn_scale = 1.0 / sqrt((double)kHeadDim);
    TL_KLAUNCH(attention_kernel, dim3(n_kv_heads, rows), dim3(256), lds, s, q8, q_scale, n_heads,
                       n_kv_heads, rm, kv, layer, kv_sk, kv_sv, attn_scale, out, dbg);
    return hipGetLastError();
}

hipError_t launch_rope(hipStream_t s, float* v, int32_t rows, int32_t n_heads, const int32_t* pos,
                       const float* cos, const float* sin) {
    if (rows <= 0) return hipSuccess;
    TL_KLAUNCH(rope_kernel, dim3(rows), dim3(256), sizeof(float) * n_heads * kHeadDim, s, v,
                       n_heads, pos, cos, sin);
    return hipGetLastError();
}

hipError_t launch_softmax_rows(hipStream_t s, const float* x, int32_t rows, int32_t n, float* p) {
    if (rows <= 0 || n <= 0) return hipSuccess;
    TL_KLAUNCH(softmax_rows_kernel, dim3(rows), dim3(256), sizeof(float) * ((n + 63) / 64), s, x, n, p);
    return hipGetLastError();
}

hipError_t launch_silu_mul(hipStream_t s, const float* g, const float* u, int64_t n, float* y) {
    if (n <= 0) return hipSuccess;
    const int blocks = (int)std::min<int64_t>(4096, (n + 255) / 256);
    TL_KLAUNCH(silu_mul_kernel, dim3(blocks), dim3(256), 0, s, g, u, n, y);
    return hipGetLastError();
}

hipError_t launch_dequant_i32(hipStream_t s, const int32_t* acc, int64_t n, int32_t cols, float m,
                              const float* bias, float* y) {
    if (n <= 0) return hipSuccess;
    const int blocks = (int)std::min<int64_t>(4096, (n + 255) / 256);
    TL_KLAUNCH(dequant_i32_kernel, dim3(blocks), dim3(256), 0, s, acc, n, cols, m, bias, y);
    return hipGetLastError();
}

hipError_t launch_fill_u32(hipStream_t s, unsigned* p, int32_t n, unsigned v) {
    if (n <= 0) return hipSuccess;
    TL_KLAUNCH(fill_u32_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, s, p, n, v);
    return hipGetLastError();
}

hipError_t launch_embed(hipStream_t s, const int32_t* tokens, int32_t rows, int32_t d, int32_t vocab,
                        const int8_t* emb, const float* emb_s, float* x) {
    if (rows <= 0) return hipSuccess;
    TL_KLAUNCH(embed_kernel, dim3(rows), dim3(256), 0, s, tokens, d, vocab, emb, emb_s, x);
    return hipGetLastError();
}

hipError_t launch_reset_keys(hipStream_t s, unsigned long long* keys, int32_t n) {
    TL_KLAUNCH(reset_keys_kernel, dim3(ceil_div(n, 64)), dim3(64), 0, s, keys, n);
    return hipGetLastError();
}

hipError_t launch_finalize_tokens(hipStream_t s, unsigned long long* keys, int32_t rows,
                                  int32_t* token_cur, int32_t* tokens_out, int32_t out_stride,
                                  int32_t* n_gen, int32_t* cursor, float* best_logit, int32_t advance,
                                  const unsigned long long* wg_keys, int32_t n_wg, EmbedNext nx) {
    if ((n_wg > 0 || nx.x) && rows != 1) return hipErrorInvalidValue;
    TL_KLAUNCH(finalize_tokens_kernel, dim3(ceil_div(rows, 64)), dim3(64), 0, s, keys, rows,
                       token_cur, tokens_out, out_stride, n_gen, cursor, best_logit, advance, wg_keys, n_wg, nx);
    return hipGetLastError();
}

hipError_t launch_argmax_rows(hipStream_t s, const float* logits, int32_t rows, int32_t n,
                              unsigned long long* keys) {
    if (rows <= 0) return hipSuccess;
    TL_KLAUNCH(argmax_rows_kernel, dim3(rows), dim3(256), 0, s, logits, n, keys);
    return hipGetLastError();
}

hipError_t init_kernels() {
    // the attention kernel keeps scores and INT8 probabilities of up to 2048
    // keys x 8 heads in LDS (gfx950: 160 KiB per workgroup)
    return hipFuncSetAttribute((const void*)attention_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                               150 * 1024);
}

hipError_t launch_step_rows(hipStream_t s, const int32_t* seq_of_row, int32_t rows,
                            const int32_t* cursor, int32_t* row_pos) {
    TL_KLAUNCH(step_rows_kernel, dim3(ceil_div(rows, 64)), dim3(64), 0, s, seq_of_row, rows,
                       cursor, row_pos);
    return hipGetLastError();
}

hipError_t launch_kv_scatter(hipStream_t s, KvGeom kv, int32_t seq, int32_t layer, int32_t g,
                             int32_t t0, int32_t n, const int8_t* k_rows, const int8_t* v_rows) {
    if (n <= 0) return hipSuccess;
    TL_KLAUNCH(kv_scatter_kernel, dim3(ceil_div((int64_t)n * kHeadDim, 256)), dim3(256), 0, s,
                       kv, kv.plane(seq, layer, g), t0, n, k_rows, v_rows);
    return hipGetLastError();
}

hipError_t launch_kv_gather(hipStream_t s, KvGeom kv, int32_t seq, int32_t layer, int32_t g,
                            int32_t t0, int32_t n, int8_t* k_rows, int8_t* v_rows) {
    if (n <= 0) return hipSuccess;
    TL_KLAUNCH(kv_gather_kernel, dim3(ceil_div((int64_t)n * kHeadDim, 256)), dim3(256), 0, s,
                       kv, kv.plane(seq, layer, g), t0, n, k_rows, v_rows);
    return hipGetLastError();
}

}  // namespace tl
