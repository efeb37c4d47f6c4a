// tl_gemm.hip -- INT8 MFMA GEMM for prefill (M = prompt length):
//   C[M][N] = A[M][K] . W[N][K]^T   (INT32, exact)   then a fused epilogue
//   (dequantization per row/channel, + residual, or SiLU(gate) * up).
//
// v_mfma_i32_32x32x32_i8: a wavefront multiplies a 32x32 A fragment by a
// 32x32 B fragment (K = 32) into 16 int32 accumulators per lane.  Each lane
// supplies 16 consecutive K bytes of one A row and of one B row: lane l holds
// row (l % 32), K bytes [(l / 32) * 16, +16); as long as A and B use the same
// lane -> K assignment the integer result is exact.  Output: lane l, register
// i holds C[8 (i / 4) + 4 (l / 32) + (i % 4)][l % 32].
//
#include <hip/hip_runtime.h>

#include <algorithm>

#include "tl_device.h"
#include "tl_internal.h"

namespace tl {

typedef int v16i __attribute__((ext_vector_type(16)));

// LDS operand tiles hold rows of BK bytes = CPR 16-byte chunks.  Chunk c of
// row r is stored at slot c ^ ((r >> S) & (CPR - 1)) with S = log2(16 / CPR):
// the 16 lanes of one LDS pass, which read the same logical chunk of 16
// consecutive rows (or write 16 chunks of the same row), then touch 16
// distinct bank quads.
template <int CPR>
TL_DEV int swz(int row, int c) {
    constexpr int S = CPR >= 16 ? 0 : (CPR == 8 ? 1 : 2);
    return row * CPR + (c ^ ((row >> S) & (CPR - 1)));
}

// WM x WN x KS wavefronts.  A wavefront owns (32 TM) x (32 TN) outputs (of
// each matrix for the GLU epilogue, which stages gate and up rows side by
// side) and one of KS interleaved K slices of every step; with KS = 2 two
// wavefronts share each SIMD, so one computes while the other waits on LDS,
// and their partial sums meet in LDS at the end.  K advances BK per step
// through a ring of three LDS buffers: while step s computes out of buffer
// s % 3, step s + 2 is written into buffer (s + 2) % 3 from one of PD
// register sets, whose global loads were issued PD steps earlier.
template <int WM, int WN, int TM, int TN, int BK, int PD, int KS>
struct GemmShape {
    static constexpr int kWaves = WM * WN * KS;
    static constexpr int kThreads = kWaves * 64;
    static constexpr int BM = 32 * TM * WM, BN = 32 * TN * WN, CPR = BK / 16;
    static constexpr int QS = BK / 32 / KS;   // 32-wide K slices per wavefront per step
};

template <int WM, int WN, int TM, int TN, int BK, int PD, int KS, int EPI>
__global__ __launch_bounds__(WM * WN * KS * 64) void gemm32_kernel(GemmArgs a) {
    using G = GemmShape<WM, WN, TM, TN, BK, PD, KS>;
    constexpr int NT = G::kThreads, BM = G::BM, BN = G::BN, CPR = G::CPR, QS = G::QS;
    constexpr int NB = (EPI == EPI_GLU) ? 2 : 1;
    constexpr int ACH = BM * CPR, BCH = BN * CPR;   // 16-byte chunks per operand tile
    static_assert(ACH % NT == 0 && BCH % NT == 0, "tile does not split evenly over threads");
    static_assert(KS == 1 || KS == 2, "one or two K slices");
    constexpr int APT = ACH / NT, BPT = BCH / NT;
    constexpr int NBUF = 3;
    constexpr int LDS_CHUNKS = NBUF * (ACH + NB * BCH);
    // the K-slice reduction reuses the operand buffers
    static_assert(KS == 1 || WM * WN * NB * TM * TN * 16 * 64 * 4 <= LDS_CHUNKS * 16, "reduction does not fit");
    __shared__ v4i lds[LDS_CHUNKS];
    auto sa = [&](int buf, int i) -> v4i& { return lds[buf * ACH + i]; };
    auto sb = [&](int buf, int b, int i) -> v4i& { return lds[NBUF * ACH + (buf * NB + b) * BCH + i]; };

    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int ks = wave / (WM * WN), wt = wave % (WM * WN);
    const int wm = wt / WN, wn = wt % WN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int kb = blockIdx.z * a.k_split;
    const int ke = min(a.k, kb + a.k_split);
    const int nfull = (ke - kb) / BK;              // full BK-wide steps
    const int wtail = (ke - kb) - nfull * BK;      // width of a final partial step (multiple of 64)
    const int nsteps = nfull + (wtail ? 1 : 0);

    // staging: chunk c = tid + NT j -> row c / CPR, K chunk c % CPR
    const int8_t* asrc[APT];
    const int8_t* bsrc[NB][BPT];
#pragma unroll
    for (int j = 0; j < APT; j++) {
        const int c = tid + NT * j;
        asrc[j] = a.a + (int64_t)min(m0 + c / CPR, a.m - 1) * a.k;
    }
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int j = 0; j < BPT; j++) {
            const int c = tid + NT * j;
            bsrc[b][j] = (b ? a.w2 : a.w) + (int64_t)min(n0 + c / CPR, a.n - 1) * a.k;
        }
    v4i ra[PD][APT], rb[PD][NB][BPT];
    auto gload = [&](int set, int step) {
        const int kk = kb + step * BK;
        // a partial last step reloads its last valid chunk in the lanes past
        // its width (in bounds)
        const int lim = (step == nfull) ? wtail - 16 : BK - 16;
#pragma unroll
        for (int j = 0; j < APT; j++) {
            const int c = tid + NT * j;
            ra[set][j] = ld16(asrc[j] + kk + min((c % CPR) * 16, lim));
        }
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int j = 0; j < BPT; j++) {
                const int c = tid + NT * j;
                rb[set][b][j] = ld16(bsrc[b][j] + kk + min((c % CPR) * 16, lim));
            }
    };
    // A partial last step (width wtail) holds reloaded bytes past its width;
    // its A chunks there are cleared in LDS, so every step can run all BK / 32
    // K slices: cleared A times any B adds exactly zero.
    auto lstore = [&](int set, int buf, int step) {
#pragma unroll
        for (int j = 0; j < APT; j++) {
            const int c = tid + NT * j;
            sa(buf, swz<CPR>(c / CPR, c % CPR)) = ra[set][j];
        }
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int j = 0; j < BPT; j++) {
                const int c = tid + NT * j;
                sb(buf, b, swz<CPR>(c / CPR, c % CPR)) = rb[set][b][j];
            }
        if (step == nfull && wtail) {
            const v4i zero = {0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < APT; j++) {
                const int c = tid + NT * j;
                if ((c % CPR) * 16 >= wtail) sa(buf, swz<CPR>(c / CPR, c % CPR)) = zero;
            }
        }
    };

    v16i acc[NB][TM][TN];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[b][i][j][e] = 0;

    const int fr = lane & 31, fk = lane >> 5;   // fragment row, 16-byte chunk inside a K=32 slice
    // all fragments of a step are read before its MFMAs start, so the LDS
    // latency of later K slices overlaps the MFMAs of earlier ones
    auto compute = [&](int buf) {
        v4i af[QS][TM], bf[QS][NB][TN];
#pragma unroll
        for (int q = 0; q < QS; q++) {
            const int kc = (ks * QS + q) * 2 + fk;
#pragma unroll
            for (int i = 0; i < TM; i++) af[q][i] = sa(buf, swz<CPR>(wm * 32 * TM + i * 32 + fr, kc));
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int j = 0; j < TN; j++) bf[q][b][j] = sb(buf, b, swz<CPR>(wn * 32 * TN + j * 32 + fr, kc));
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < QS; q++)
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[b][i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[q][i], bf[q][b][j], acc[b][i][j], 0, 0, 0);
    };
    // step s: write step s + 2 (register set (s + 2) % PD) into LDS buffer
    // (s + 2) % 3, whose last reader, step s - 1, finished at the previous
    // barrier; reload that register set with step s + 2 + PD; compute step s
    // from buffer s % 3, written two steps ago; barrier.  Loads, LDS stores
    // and barriers do not depend on data: the step index of a load past the
    // end is clamped to the last step (a redundant, in-bounds reload; steps
    // past the end are written to LDS but never read), so the wait before
    // each LDS store covers exactly one step's loads and the PD - 1 steps
    // after it stay in flight.
    auto step = [&](int s, int u) {
        const int set = (u + 2) % PD;
        lstore(set, (s + 2) % NBUF, s + 2);
        gload(set, min(s + 2 + PD, nsteps - 1));
        compute(s % NBUF);
        __syncthreads();
    };
    if (nsteps > 0) {
#pragma unroll
        for (int u = 0; u < PD; u++) gload(u, min(u, nsteps - 1));
        lstore(0, 0, 0);
        gload(0, min(PD, nsteps - 1));
        lstore(1 % PD, 1, 1);
        gload(1 % PD, min(PD + 1, nsteps - 1));
        __syncthreads();
        int s0 = 0;
        for (; s0 + PD <= nsteps; s0 += PD) {
#pragma unroll
            for (int u = 0; u < PD; u++) step(s0 + u, u);
        }
#pragma unroll
        for (int u = 0; u < PD - 1; u++)
            if (s0 + u < nsteps) step(s0 + u, u);
    }

    if (KS == 2) {
        // the last step ended with a barrier: LDS is free.  Slice 1 parks its
        // partial sums (lane-contiguous), slice 0 adds them and runs the
        // epilogue.
        int* red = reinterpret_cast<int*>(lds);
        if (ks == 1) {
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
#pragma unroll
                        for (int e = 0; e < 16; e++)
                            red[(((wt * NB + b) * TM + i) * TN + j) * 1024 + e * 64 + lane] = acc[b][i][j][e];
        }
        __syncthreads();
        if (ks == 1) return;
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
#pragma unroll
                    for (int e = 0; e < 16; e++)
                        acc[b][i][j][e] += red[(((wt * NB + b) * TM + i) * TN + j) * 1024 + e * 64 + lane];
    }

    // epilogue.  Lane l, register e of a 32 x 32 block holds row
    // 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32.  Every load (row and
    // channel scales, residual) is issued before the first store: the output
    // could alias them as far as the compiler knows, and loads ordered after
    // stores would cost one cache round trip per element.
    const bool partial = gridDim.z > 1 || EPI == EPI_RAW;
    const int64_t plane = (int64_t)a.m * a.n;
    const int rbase = m0 + wm * 32 * TM + 4 * (lane >> 5);
    const int cbase = n0 + wn * 32 * TN + (lane & 31);
    if (partial) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int n = cbase + j * 32;
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int m = rbase + i * 32 + 8 * (e >> 2) + (e & 3);
                    if (m < a.m && n < a.n)
#pragma unroll
                        for (int b = 0; b < NB; b++)
                            a.acc[(int64_t)(blockIdx.z * NB + b) * plane + (int64_t)m * a.n + n] = acc[b][i][j][e];
                }
            }
        return;
    }
    double sx[TM][16];
    float sw[NB][TN];
    float res[TM][TN][EPI == EPI_DEQUANT_RES ? 16 : 1];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) sx[i][e] = a.as[min(rbase + i * 32 + 8 * (e >> 2) + (e & 3), a.m - 1)];
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = min(cbase + j * 32, a.n - 1);
        sw[0][j] = a.ws[n];
        if (EPI == EPI_GLU) sw[NB - 1][j] = a.ws2[n];
    }
    if (EPI == EPI_DEQUANT_RES) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int m = min(rbase + i * 32 + 8 * (e >> 2) + (e & 3), a.m - 1);
                    res[i][j][e] = a.residual[(int64_t)m * a.n + min(cbase + j * 32, a.n - 1)];
                }
    }
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = cbase + j * 32;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int m = rbase + i * 32 + 8 * (e >> 2) + (e & 3);
                const float v0 = (float)acc[0][i][j][e] * deq_mult(sx[i][e], sw[0][j]);
                float out;
                if (EPI == EPI_GLU) {
                    const float up = (float)acc[NB - 1][i][j][e] * deq_mult(sx[i][e], sw[NB - 1][j]);
                    out = tl_silu(v0) * up;
                } else if (EPI == EPI_DEQUANT_RES) {
                    out = res[i][j][e] + v0;
                } else {
                    out = v0;
                }
                if (m < a.m && n < a.n) a.y[(int64_t)m * a.n + n] = out;
            }
        }
}

// ---------------------------------------------------------------------------
// Block-tiled GEMM for prefill-sized M: WM x WN wavefronts, each owning
// TM x TN blocks of 32 x 32 outputs (of each matrix for the GLU epilogue).
// K advances BK bytes per stage through two LDS buffers with one barrier per
// stage, so a wavefront issues BK / 32 x TM x TN x NB MFMAs between barriers
// (16 at the 2 x 2 blocks and BK = 128 of the default).  Global loads run PD
// stages ahead in register sets: stage k + PD is loaded while stage k
// computes.  Every fragment of a stage is read from LDS before its MFMAs.
// ---------------------------------------------------------------------------
template <int WM, int WN, int TM, int TN, int BK, int PD, int EPI>
__global__ __launch_bounds__(WM * WN * 64) void gemm_tile_kernel(GemmArgs a) {
    constexpr int NT = WM * WN * 64, BM = 32 * TM * WM, BN = 32 * TN * WN, CPR = BK / 16, SL = BK / 32;
    constexpr int NB = (EPI == EPI_GLU) ? 2 : 1;
    constexpr int ACH = BM * CPR, BCH = BN * CPR;   // 16-byte chunks per operand tile
    static_assert(ACH % NT == 0 && BCH % NT == 0, "tile does not split evenly over threads");
    constexpr int APT = ACH / NT, BPT = BCH / NT;
    constexpr int STAGE = ACH + NB * BCH;            // chunks per LDS buffer
    __shared__ v4i lds[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int wm = wave / WN, wn = wave % WN;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int nk = a.k / BK;

    // staging: chunk c = tid + NT j -> row c / CPR, K chunk c % CPR
    const int8_t* asrc[APT];
    const int8_t* bsrc[NB][BPT];
#pragma unroll
    for (int j = 0; j < APT; j++) {
        const int c = tid + NT * j;
        asrc[j] = a.a + (int64_t)min(m0 + c / CPR, a.m - 1) * a.k + (c % CPR) * 16;
    }
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int j = 0; j < BPT; j++) {
            const int c = tid + NT * j;
            bsrc[b][j] = (b ? a.w2 : a.w) + (int64_t)min(n0 + c / CPR, a.n - 1) * a.k + (c % CPR) * 16;
        }
    v4i ra[PD][APT], rb[PD][NB][BPT];
    auto gload = [&](int set, int stage) {
        const int kk = stage * BK;
#pragma unroll
        for (int j = 0; j < APT; j++) ra[set][j] = ld16(asrc[j] + kk);
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int j = 0; j < BPT; j++) rb[set][b][j] = ld16(bsrc[b][j] + kk);
    };
    auto lstore = [&](int set, int buf) {
        v4i* base = lds + buf * STAGE;
#pragma unroll
        for (int j = 0; j < APT; j++) {
            const int c = tid + NT * j;
            base[swz<CPR>(c / CPR, c % CPR)] = ra[set][j];
        }
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int j = 0; j < BPT; j++) {
                const int c = tid + NT * j;
                base[ACH + b * BCH + swz<CPR>(c / CPR, c % CPR)] = rb[set][b][j];
            }
    };

    v16i acc[NB][TM][TN];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[b][i][j][e] = 0;

    const int fr = lane & 31, fk = lane >> 5;   // fragment row, 16-byte chunk inside a 32-byte K slice
    auto compute = [&](int buf) {
        const v4i* base = lds + buf * STAGE;
        v4i af[SL][TM], bf[SL][NB][TN];
#pragma unroll
        for (int q = 0; q < SL; q++) {
            const int kc = q * 2 + fk;
#pragma unroll
            for (int i = 0; i < TM; i++) af[q][i] = base[swz<CPR>(wm * 32 * TM + i * 32 + fr, kc)];
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int j = 0; j < TN; j++) bf[q][b][j] = base[ACH + b * BCH + swz<CPR>(wn * 32 * TN + j * 32 + fr, kc)];
        }
#pragma unroll
        for (int q = 0; q < SL; q++)
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[b][i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[q][i], bf[q][b][j], acc[b][i][j], 0, 0, 0);
    };

    // stage k: store register set k % PD into buffer k % 2 (its last reader,
    // stage k - 2, finished before the barrier of stage k - 1), reload the set
    // with stage k + PD (clamped: a redundant in-bounds reload past the end),
    // barrier, compute
#pragma unroll
    for (int u = 0; u < PD; u++) gload(u, min(u, nk - 1));
    int k = 0;
    for (; k + PD <= nk; k += PD) {
#pragma unroll
        for (int u = 0; u < PD; u++) {
            lstore(u, (k + u) & 1);
            gload(u, min(k + u + PD, nk - 1));
            __syncthreads();
            compute((k + u) & 1);
        }
    }
#pragma unroll
    for (int u = 0; u < PD; u++) {
        if (k + u < nk) {
            lstore(u, (k + u) & 1);
            __syncthreads();
            compute((k + u) & 1);
        }
    }

    // epilogue (lane l, register e of a 32 x 32 block: row 8 (e / 4) +
    // 4 (l / 32) + e % 4, column l % 32); all loads before the first store
    const int rbase = m0 + wm * 32 * TM + 4 * (lane >> 5);
    const int cbase = n0 + wn * 32 * TN + (lane & 31);
    if (EPI == EPI_RAW) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int n = cbase + j * 32;
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int m = rbase + i * 32 + 8 * (e >> 2) + (e & 3);
                    if (m < a.m && n < a.n) a.acc[(int64_t)m * a.n + n] = acc[0][i][j][e];
                }
            }
        return;
    }
    double sx[TM][16];
    float sw[NB][TN];
    float res[TM][TN][EPI == EPI_DEQUANT_RES ? 16 : 1];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) sx[i][e] = a.as[min(rbase + i * 32 + 8 * (e >> 2) + (e & 3), a.m - 1)];
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = min(cbase + j * 32, a.n - 1);
        sw[0][j] = a.ws[n];
        if (EPI == EPI_GLU) sw[NB - 1][j] = a.ws2[n];
    }
    if (EPI == EPI_DEQUANT_RES) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int m = min(rbase + i * 32 + 8 * (e >> 2) + (e & 3), a.m - 1);
                    res[i][j][e] = a.residual[(int64_t)m * a.n + min(cbase + j * 32, a.n - 1)];
                }
    }
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = cbase + j * 32;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int m = rbase + i * 32 + 8 * (e >> 2) + (e & 3);
                const float v0 = (float)acc[0][i][j][e] * deq_mult(sx[i][e], sw[0][j]);
                float out;
                if (EPI == EPI_GLU) {
                    const float up = (float)acc[NB - 1][i][j][e] * deq_mult(sx[i][e], sw[NB - 1][j]);
                    out = tl_silu(v0) * up;
                } else if (EPI == EPI_DEQUANT_RES) {
                    out = res[i][j][e] + v0;
                } else {
                    out = v0;
                }
                if (m < a.m && n < a.n) a.y[(int64_t)m * a.n + n] = out;
            }
        }
}

// Row-major operands (the tl_gemm_i8 operator, and prefill shapes the packed
// path does not take), M >= 64, 32x32x32 MFMA tiles:
//   gemm_tile_kernel, K a multiple of 128: 2 x 2 wavefronts of one 32 x 32
//     block each (64 x 64 block tile), 128-byte K stages through two LDS
//     buffers, four register sets;
//   gemm32_kernel otherwise: 2 x 2 x 2 wavefronts (the K slice split in two
//     inside the workgroup), 64 x 64 block tile, three register sets.
// At M = 512 the 64 x 64 tiles measured fastest; larger block tiles leave CUs
// idle at these N.
template <int WM, int WN, int TM, int TN, int BK, int PD, int KS, int EPI>
static void go32(hipStream_t s, const GemmArgs& a, int32_t splits) {
    using G = GemmShape<WM, WN, TM, TN, BK, PD, KS>;
    const dim3 grid((a.n + G::BN - 1) / G::BN, (a.m + G::BM - 1) / G::BM, splits);
    TL_KLAUNCH((gemm32_kernel<WM, WN, TM, TN, BK, PD, KS, EPI>), grid, dim3(G::kThreads), 0, s, a);
}

template <int WM, int WN, int TM, int TN, int BK, int PD, int EPI>
static bool go_tile(hipStream_t s, const GemmArgs& a) {
    constexpr int BM = 32 * TM * WM, BN = 32 * TN * WN;
    if (a.k % BK) return false;
    const dim3 grid((a.n + BN - 1) / BN, (a.m + BM - 1) / BM, 1);
    TL_KLAUNCH((gemm_tile_kernel<WM, WN, TM, TN, BK, PD, EPI>), grid, dim3(WM * WN * 64), 0, s, a);
    return true;
}

template <int EPI>
static bool shape32(hipStream_t s, const GemmArgs& a, bool tile) {
    if (tile) return go_tile<2, 2, 1, 1, 128, 4, EPI>(s, a);
    go32<2, 2, 1, 1, 128, 3, 2, EPI>(s, a, 1);
    return true;
}

// M >= 64, row-major operands, the whole K in one launch: gemm_tile_kernel
// (tile; K a multiple of 128) or gemm32_kernel
hipError_t launch_gemm32(hipStream_t s, int epi, const GemmArgs& args, bool tile) {
    GemmArgs a = args;
    if (a.m <= 0 || a.n <= 0) return hipSuccess;
    if (a.k <= 0 || a.k % 64 != 0 || (tile && a.k % 128)) return hipErrorInvalidValue;
    a.k_split = a.k;
    bool ok = false;
    switch (epi) {
        case EPI_DEQUANT: ok = shape32<EPI_DEQUANT>(s, a, tile); break;
        case EPI_DEQUANT_RES: ok = shape32<EPI_DEQUANT_RES>(s, a, tile); break;
        case EPI_GLU: ok = shape32<EPI_GLU>(s, a, tile); break;
        case EPI_RAW: ok = shape32<EPI_RAW>(s, a, tile); break;
        default: break;
    }
    if (!ok) return hipErrorInvalidValue;
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Prefill GEMMs on packed operands (a.ap, a.wp, a.wp2).  Both operands are
// stored as 1 KiB MFMA blocks: block (t, c) holds rows [32 t, 32 t + 32) x K
// bytes [32 c, 32 c + 32), with row 32 t + l % 32's K bytes 32 c + 16 (l / 32)
// .. +16 at byte 16 l, so a wavefront's fragment load is one coalesced 1 KiB
// read that hands lane l exactly its MFMA operand.  A's rows are padded to
// the row tile (128); what the padding rows hold only reaches discarded rows.
//
// Why this form (measured at M = 512, TinyLlama shapes): a CU takes in about
// 33 bytes per clock through its vector loads, whether they land in
// registers or in LDS (global -> LDS loads), and loads that feed LDS add to
// the fragment reads out of LDS instead of overlapping them.  So fragments
// that one wavefront alone uses go straight into its registers, and only
// operands that several wavefronts share go through LDS.
// ---------------------------------------------------------------------------

typedef __attribute__((address_space(1))) void PkGlobal;
typedef __attribute__((address_space(3))) void PkLds;

TL_DEV const int8_t* pk_block(const int8_t* base, int tile, int chunk, int kc) {
    return base + ((int64_t)tile * kc + chunk) * 1024;
}

template <int N_>
TL_DEV void pk_wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N_) : "memory");
}

// the same wait, taking the four registers of an asm-issued fragment load as
// operands: whatever reads them is ordered after the wait
template <int N_>
TL_DEV void pk_wait_regs(v4i* r) {
    asm volatile("s_waitcnt vmcnt(%4)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]) : "n"(N_));
}

// (1) one-matrix GEMMs (DEQUANT, DEQUANT_RES), K a multiple of 512: the 4
// wavefronts of a workgroup each compute the whole (32 TM) x (32 TN) tile
// over their own quarter of K, both operands straight into registers
// kPkSplitPD chunks (of 32 K bytes) ahead, with no LDS and no barrier in the
// main loop.  The four partial tiles are added through LDS (exact integers)
// and wavefront w finishes blocks w, w + 4, ... of the tile with the epilogue
// arithmetic of every other GEMM here.  Tiles: 64 x 64 (TM = TN = 2) for O and
// down (256 workgroups at M = 512), 32 x 160 (TM = 1, TN = 5) for Q|K|V
// (N = 2560: 256 workgroups where 64 x 64 needs 320); 64 x 64 for the
// prefill Q|K|V with qkv_post's work in the epilogue (EPI_QKV_ROPE, one head
// per tile).  The epilogue's operands are loaded behind the last operand
// loads, so they arrive during the last MFMAs.
constexpr int kPkSplitPD = 4;

static size_t pk_split_lds_bytes(int tm, int tn) { return (size_t)4 * tm * tn * 16 * 64 * sizeof(int); }

// EPI_QKV_ROPE epilogue of a 64 x 64 tile (one head of Q, K or V): wavefront
// w takes accumulator registers 8 (w % 2) .. 8 (w % 2) + 7 (8 rows per lane) of
// row block w / 2 in both column blocks, so a lane holds dimensions d and
// d + 32 of its rows.  The
// arithmetic is qkv_post_kernel's: x = f32(acc) f32(sx sw), rotated
// x_d c_d + (-x_{d+32}) s_d and x_{d+32} c_{d+32} + x_d s_{d+32} (two products
// and a sum, no fused multiply-add), K and V bytes sat(rne(x / s)).  Its
// operands (row scales, positions, sequences, cos / sin) are loaded before
// the LDS reduction (qkv_rope_operands, qkv_rope_tables).
struct QkvRopeOps {   // the 8 registers (rows) of the wavefront's row block
    double sx[8];
    int pos[8], seq[8];
    float c0[8], s0[8], c1[8], s1[8];
    float sw0, sw1, sc;
    int region, g, n0, rb, e0, i;
};

TL_DEV void qkv_rope_operands(const GemmArgs& a, const QkvRopeArgs& f, int mt0, int nt0, int wave, int lane,
                              QkvRopeOps& o) {
    constexpr int NE = 8;
    const int d = lane & 31, D = f.n_heads * kHeadDim, KVD = f.n_kv * kHeadDim;
    o.i = wave >> 1;
    o.e0 = (wave & 1) * 8;
    o.n0 = nt0 * 32;
    o.region = o.n0 < D ? 0 : (o.n0 < D + KVD ? 1 : 2);   // Q, K, V (uniform)
    o.g = o.region == 1 ? (o.n0 - D) >> 6 : (o.n0 - D - KVD) >> 6;
    o.rb = (mt0 + o.i) * 32 + 4 * (lane >> 5);
    o.sw0 = a.ws[o.n0 + d];
    o.sw1 = a.ws[o.n0 + 32 + d];
    o.sc = o.region == 1 ? f.kv_sk[f.layer * f.n_kv + o.g] : (o.region == 2 ? f.kv_sv[f.layer * f.n_kv + o.g] : 1.0f);
#pragma unroll
    for (int ee = 0; ee < NE; ee++) {
        const int e = o.e0 + ee, m = min(o.rb + 8 * (e >> 2) + (e & 3), a.m - 1);
        o.sx[ee] = a.as[m];
        o.pos[ee] = f.rm.pos[m];
        o.seq[ee] = f.rm.seq[m];
    }
}

// the cos / sin entries of the rows' positions (after qkv_rope_operands)
TL_DEV void qkv_rope_tables(const QkvRopeArgs& f, int lane, QkvRopeOps& o) {
    constexpr int NE = 8;
    const int d = lane & 31;
    if (o.region != 2) {
#pragma unroll
        for (int ee = 0; ee < NE; ee++) {
            const int64_t t = (int64_t)min(max(o.pos[ee], 0), f.kv.max_pos - 1) * kHeadDim;
            o.c0[ee] = f.cosb[t + d];
            o.s0[ee] = f.sinb[t + d];
            o.c1[ee] = f.cosb[t + d + 32];
            o.s1[ee] = f.sinb[t + d + 32];
        }
    }
}

TL_DEV void qkv_rope_epilogue(const GemmArgs& a, const QkvRopeArgs& f, const QkvRopeOps& o, const int* red,
                              int lane) {
    constexpr int NBLK = 4, NE = 8;
    const int d = lane & 31, D = f.n_heads * kHeadDim;
    int a0[NE], a1[NE];   // every partial sum first: the LDS reads overlap
#pragma unroll
    for (int ee = 0; ee < NE; ee++) {
        const int e = o.e0 + ee;
        a0[ee] = 0;
        a1[ee] = 0;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            a0[ee] += red[((w * NBLK + o.i * 2) * 16 + e) * 64 + lane];
            a1[ee] += red[((w * NBLK + o.i * 2 + 1) * 16 + e) * 64 + lane];
        }
    }
#pragma unroll
    for (int ee = 0; ee < NE; ee++) {
        const int e = o.e0 + ee, m = o.rb + 8 * (e >> 2) + (e & 3);
        const float lo = (float)a0[ee] * deq_mult(o.sx[ee], o.sw0), hi = (float)a1[ee] * deq_mult(o.sx[ee], o.sw1);
        const int pos = o.pos[ee];
        const bool valid = m < a.m && pos >= 0 && pos < f.kv.max_pos;   // uniform per half-wavefront
        if (o.region == 2) {
            if (valid) {
                const int64_t pl = f.kv.plane(o.seq[ee], f.layer, o.g);
                f.kv.v[pl + KvGeom::v_off(pos, d)] = sat_i8(__builtin_rintf(__fdiv_rn(lo, o.sc)));
                f.kv.v[pl + KvGeom::v_off(pos, d + 32)] = sat_i8(__builtin_rintf(__fdiv_rn(hi, o.sc)));
            }
            continue;
        }
        const float rlo = (lo * o.c0[ee]) + ((-hi) * o.s0[ee]);
        const float rhi = (hi * o.c1[ee]) + (lo * o.s1[ee]);
        if (o.region == 1) {
            if (valid) {
                const int64_t pl = f.kv.plane(o.seq[ee], f.layer, o.g);
                f.kv.k[pl + KvGeom::k_off(pos, d)] = sat_i8(__builtin_rintf(__fdiv_rn(rlo, o.sc)));
                f.kv.k[pl + KvGeom::k_off(pos, d + 32)] = sat_i8(__builtin_rintf(__fdiv_rn(rhi, o.sc)));
            }
            continue;
        }
        if (m < a.m) {
            f.q_out[(int64_t)m * D + o.n0 + d] = rlo;
            f.q_out[(int64_t)m * D + o.n0 + d + 32] = rhi;
        }
        const float mx = half_max_f32(valid ? fmaxf(fabsf(rlo), fabsf(rhi)) : 0.0f);   // the row's 32 lanes
        if (d == 0 && valid) atomicMax(f.q_max + (int64_t)m * kQmaxStride, __float_as_uint(mx));
    }
}

// operands of the DEQUANT(_RES) epilogue of the blocks wavefront w finishes
// (w, w + 4, ...: NBW at most), loaded before the main loop
template <int NBW, bool RES>
struct SplitOps {
    double sx[NBW][16];
    float res[NBW][RES ? 16 : 1];
    float sw[NBW];
};

template <int TM, int TN, int EPI>
__global__ __launch_bounds__(256) void gemm_pk_split_kernel(GemmArgs a, QkvRopeArgs f) {
    constexpr int NF = TM + TN, PD = kPkSplitPD, NBLK = TM * TN, NBW = (NBLK + 3) / 4;
    constexpr bool RES = EPI == EPI_DEQUANT_RES;
    extern __shared__ __align__(16) int pk_red[];   // [4 waves][NBLK][16][64]
    const int kc = a.k >> 5, per = kc >> 2;        // chunks of each wavefront (a multiple of PD)
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int mt0 = blockIdx.y * TM, nt0 = blockIdx.x * TN, c0 = wave * per;
    const int8_t* ab = a.ap + lane * 16;
    const int8_t* wb = a.wp + lane * 16;
    v4i r[PD][NF];
    auto load = [&](int set, int c) {
#pragma unroll
        for (int i = 0; i < TM; i++) r[set][i] = ld16(pk_block(ab, mt0 + i, c, kc));
#pragma unroll
        for (int j = 0; j < TN; j++) r[set][TM + j] = ld16(pk_block(wb, nt0 + j, c, kc));
    };
    v16i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = (v16i){};
    auto mma = [&](int set) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(r[set][i], r[set][TM + j], acc[i][j], 0, 0, 0);
    };
    // register set u holds chunks u, u + PD, ...: the loop body reloads each
    // set right after its MFMAs, unconditionally (the last PD chunks are
    // peeled), so every wait is for the oldest set only
#pragma unroll
    for (int u = 0; u < PD; u++) load(u, c0 + u);
    int c = PD;
    for (; c < per - PD; c += PD) {
#pragma unroll
        for (int u = 0; u < PD; u++) {
            mma(u);
            load(u, c0 + c + u);
        }
    }
    if (c < per) {   // the last reloads
#pragma unroll
        for (int u = 0; u < PD; u++) {
            mma(u);
            load(u, c0 + c + u);
        }
    }
    // the epilogue's operands go out behind the last operand loads: their
    // latency passes under the last PD sets of MFMAs instead of after them
    // (vector-memory waits complete in issue order, so issued earlier they
    // would hold up the main loop's waits).  Block b, lane l, register e is
    // output row 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32.
    QkvRopeOps qo;
    SplitOps<NBW, RES> so;
    if constexpr (EPI == EPI_QKV_ROPE) {
        static_assert(TM == 2 && TN == 2, "one 64-row x one-head tile");
        qkv_rope_operands(a, f, mt0, nt0, wave, lane, qo);
    } else {
#pragma unroll
        for (int bw = 0; bw < NBW; bw++) {
            const int b = min(wave + 4 * bw, NBLK - 1);
            const int i = b / TN, j = b % TN, n = (nt0 + j) * 32 + (lane & 31);
            const int rb = (mt0 + i) * 32 + 4 * (lane >> 5);
            so.sw[bw] = a.ws[n];
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int m = min(rb + 8 * (e >> 2) + (e & 3), a.m - 1);
                so.sx[bw][e] = a.as[m];
                if constexpr (RES) so.res[bw][e] = a.residual[(int64_t)m * a.n + n];
            }
        }
    }
#pragma unroll
    for (int u = 0; u < PD; u++) mma(u);
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) pk_red[((wave * NBLK + i * TN + j) * 16 + e) * 64 + lane] = acc[i][j][e];
    if constexpr (EPI == EPI_QKV_ROPE) qkv_rope_tables(f, lane, qo);
    __syncthreads();
    if constexpr (EPI == EPI_QKV_ROPE) {
        qkv_rope_epilogue(a, f, qo, pk_red, lane);
        return;
    }
    // wavefront w finishes blocks w, w + 4, ... (y may be the residual, read
    // above and written here in place).  Every partial sum is read before
    // any store, outside the row test, so the LDS reads overlap instead of
    // paying one LDS round trip per element.
#pragma unroll
    for (int bw = 0; bw < NBW; bw++) {
        const int b = wave + 4 * bw;
        if (b >= NBLK) break;
        const int i = b / TN, j = b % TN, n = (nt0 + j) * 32 + (lane & 31);
        const int rb = (mt0 + i) * 32 + 4 * (lane >> 5);
        int sum[16];
#pragma unroll
        for (int e = 0; e < 16; e++) {
            sum[e] = 0;
#pragma unroll
            for (int w = 0; w < 4; w++) sum[e] += pk_red[((w * NBLK + b) * 16 + e) * 64 + lane];
        }
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int m = rb + 8 * (e >> 2) + (e & 3);
            const float v = (float)sum[e] * deq_mult(so.sx[bw][e], so.sw[bw]);
            if (m < a.m) a.y[(int64_t)m * a.n + n] = RES ? so.res[bw][RES ? e : 0] + v : v;
        }
    }
}

// (2) the GLU GEMM (gate and up), K a multiple of 256: 128 x (32 TN) output
// tiles of each matrix, 4 x 1 wavefronts.  Wavefront w owns rows
// [32 w, 32 w + 32) of the tile: its A fragments are its own and go straight
// into registers two 128-byte K stages ahead.  The 8 TN weight blocks of a
// stage (2 matrices x TN column tiles x 4 K chunks) are shared by the 4
// wavefronts and arrive by global -> LDS loads (2 TN per wavefront) in a ring
// of three stage buffers with one barrier per stage: stage k + 2 is loaded
// into the buffer stage k - 1 used.  __syncthreads would wait for every
// global -> LDS load in flight (they count as LDS writes to its fence), so the
// barrier is a bare s_barrier after an explicit wait for this wavefront's
// loads of the stage.  The SiLU-GLU epilogue runs on the wavefront's own
// accumulators.
constexpr int kPkGluStages = 3;

static size_t pk_glu_lds_bytes(int tn) { return (size_t)kPkGluStages * 8 * tn * 1024; }

// the stage's 8 TN weight fragments (block (s TN + j) 4 + q at byte 1024 x
// block from addr) by one asm block that ends in its own LDS wait: the
// compiler would otherwise make every LDS read wait for all global -> LDS
// loads in flight, as it cannot tell the ring's buffers apart.  `keep` are
// registers that must not be reused for the results (the addresses of the
// global -> LDS loads just issued).
template <int TN>
TL_DEV void pk_lds_frags(v4i* bq, uint32_t addr, const int8_t* const* keep) {
    if constexpr (TN == 1) {
        asm volatile(
            "ds_read_b128 %0, %8\n\tds_read_b128 %1, %8 offset:1024\n\t"
            "ds_read_b128 %2, %8 offset:2048\n\tds_read_b128 %3, %8 offset:3072\n\t"
            "ds_read_b128 %4, %8 offset:4096\n\tds_read_b128 %5, %8 offset:5120\n\t"
            "ds_read_b128 %6, %8 offset:6144\n\tds_read_b128 %7, %8 offset:7168\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(bq[0]), "=&v"(bq[1]), "=&v"(bq[2]), "=&v"(bq[3]), "=&v"(bq[4]), "=&v"(bq[5]), "=&v"(bq[6]),
              "=&v"(bq[7])
            : "v"(addr), "v"(keep[0]), "v"(keep[1]));
    } else {
        asm volatile(
            "ds_read_b128 %0, %16\n\tds_read_b128 %1, %16 offset:1024\n\t"
            "ds_read_b128 %2, %16 offset:2048\n\tds_read_b128 %3, %16 offset:3072\n\t"
            "ds_read_b128 %4, %16 offset:4096\n\tds_read_b128 %5, %16 offset:5120\n\t"
            "ds_read_b128 %6, %16 offset:6144\n\tds_read_b128 %7, %16 offset:7168\n\t"
            "ds_read_b128 %8, %16 offset:8192\n\tds_read_b128 %9, %16 offset:9216\n\t"
            "ds_read_b128 %10, %16 offset:10240\n\tds_read_b128 %11, %16 offset:11264\n\t"
            "ds_read_b128 %12, %16 offset:12288\n\tds_read_b128 %13, %16 offset:13312\n\t"
            "ds_read_b128 %14, %16 offset:14336\n\tds_read_b128 %15, %16 offset:15360\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(bq[0]), "=&v"(bq[1]), "=&v"(bq[2]), "=&v"(bq[3]), "=&v"(bq[4]), "=&v"(bq[5]), "=&v"(bq[6]),
              "=&v"(bq[7]), "=&v"(bq[8]), "=&v"(bq[9]), "=&v"(bq[10]), "=&v"(bq[11]), "=&v"(bq[12]),
              "=&v"(bq[13]), "=&v"(bq[14]), "=&v"(bq[15])
            : "v"(addr), "v"(keep[0]), "v"(keep[1]), "v"(keep[2]), "v"(keep[3]));
    }
}

template <int TN>
__global__ __launch_bounds__(256) void gemm_pk_glu_kernel(GemmArgs a) {
    constexpr int NB = 2, BB = 8 * TN, PWB = BB / 4, NS = kPkGluStages;
    extern __shared__ __align__(16) int8_t pk_glu_lds[];   // [NS][BB][1024]
    const int kc = a.k >> 5, nk = a.k >> 7;                 // 128-byte stages, an even count >= 2
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int mt = blockIdx.y * 4 + wave, nt0 = blockIdx.x * TN;
    const int8_t* ab = a.ap + lane * 16;
    // The A fragment loads are issued from inline asm and waited for by
    // explicit vmcnt counts that follow the issue order below: the compiler,
    // seeing register loads and global -> LDS loads in flight together, would
    // wait for all of them before each stage's MFMAs.  A wait takes the
    // registers it guards as operands, so nothing reads them before it; the
    // LDS fragment reads are asm too, so the compiler has no LDS read to
    // order after the global -> LDS loads.
    v4i ra[2][4];
    auto a_load = [&](int set, int stage) {
#pragma unroll
        for (int q = 0; q < 4; q++)
            asm volatile("global_load_dwordx4 %0, %1, off"
                         : "=v"(ra[set][q])
                         : "v"(pk_block(ab, mt, stage * 4 + q, kc)));
    };
    const int8_t* src[PWB];   // this stage's global -> LDS sources
#pragma unroll
    for (int j = 0; j < PWB; j++) src[j] = a.wp;
    auto b_issue = [&](int stage, int buf) {
#pragma unroll
        for (int j = 0; j < PWB; j++) {
            const int b = wave * PWB + j, mat = b / (TN * 4), bb = b % (TN * 4);
            src[j] = pk_block(mat ? a.wp2 : a.wp, nt0 + bb / 4, stage * 4 + bb % 4, kc) + lane * 16;
            __builtin_amdgcn_global_load_lds((PkGlobal*)src[j], (PkLds*)(pk_glu_lds + (buf * BB + b) * 1024), 16, 0, 0);
        }
    };
    v16i acc[NB][TN];
#pragma unroll
    for (int s = 0; s < NB; s++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[s][j] = (v16i){};
    auto compute = [&](int kk, int u) {
        v4i bq[BB];
        pk_lds_frags<TN>(bq, (uint32_t)(uintptr_t)(pk_glu_lds + (kk % NS) * BB * 1024 + lane * 16), src);
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int s = 0; s < NB; s++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[s][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ra[u][q], bq[(s * TN + j) * 4 + q], acc[s][j], 0, 0, 0);
    };
    // issue order: B(0) A(0) B(1) A(1), then per stage kk: B(kk + 2) ... A(kk + 2).
    // Stage kk: B(kk) is done when at most A(kk), B(kk + 1), A(kk + 1) remain
    // (PWB + 8); after the barrier every wavefront's is, and every wavefront
    // is past stage kk - 1, whose buffer takes B(kk + 2); A(kk) is done when
    // at most B(kk + 1), A(kk + 1), B(kk + 2) remain (2 PWB + 4).
    b_issue(0, 0);
    a_load(0, 0);
    b_issue(1, 1);
    a_load(1, 1);
    for (int k = 0; k < nk - 2; k += 2) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int kk = k + u;
            pk_wait_vm<PWB + 8>();
            asm volatile("s_barrier" ::: "memory");
            b_issue(kk + 2, (kk + 2) % NS);
            pk_wait_regs<2 * PWB + 4>(ra[u]);
            compute(kk, u);
            a_load(u, kk + 2);
        }
    }
    // the last two stages issue nothing: B(nk - 2) waits on A(nk - 2),
    // B(nk - 1), A(nk - 1); A(nk - 2) on B(nk - 1), A(nk - 1); B(nk - 1) on
    // A(nk - 1); A(nk - 1) on nothing
    pk_wait_vm<PWB + 8>();
    asm volatile("s_barrier" ::: "memory");
    pk_wait_regs<PWB + 4>(ra[0]);
    compute(nk - 2, 0);
    pk_wait_vm<4>();
    asm volatile("s_barrier" ::: "memory");
    pk_wait_regs<0>(ra[1]);
    compute(nk - 1, 1);
    const int rb = mt * 32 + 4 * (lane >> 5);
    double sx[16];
#pragma unroll
    for (int e = 0; e < 16; e++) sx[e] = a.as[min(rb + 8 * (e >> 2) + (e & 3), a.m - 1)];
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = (nt0 + j) * 32 + (lane & 31);
        const float sg = a.ws[n], su = a.ws2[n];
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int m = rb + 8 * (e >> 2) + (e & 3);
            const float gt = (float)acc[0][j][e] * deq_mult(sx[e], sg);
            const float up = (float)acc[1][j][e] * deq_mult(sx[e], su);
            if (m < a.m) a.y[(int64_t)m * a.n + n] = tl_silu(gt) * up;
        }
    }
}

// tile of the one-matrix packed GEMM: 32 x 160 when N is a multiple of 160
// and that covers the chip in fewer rounds of 256 workgroups than 64 x 64
static bool pk_split_narrow(int32_t m, int32_t n) {
    if (n % 160) return false;
    const int64_t t22 = (int64_t)((m + 63) / 64) * (n / 64), t15 = (int64_t)((m + 31) / 32) * (n / 160);
    return n % 64 != 0 || (t15 + 255) / 256 < (t22 + 255) / 256;
}

bool gemm_pk_supported(int epi, int32_t m, int32_t n, int32_t k) {
    if (m < 1 || n < 1 || k < 1) return false;
    if (epi == EPI_GLU) return n % 64 == 0 && k % 256 == 0;   // both tile widths
    if (epi != EPI_DEQUANT && epi != EPI_DEQUANT_RES) return false;
    return k % 512 == 0 && (n % 64 == 0 || pk_split_narrow(m, n));
}

int32_t gemm_pk_row_pad() { return 128; }

hipError_t launch_gemm_pk(hipStream_t s, int epi, const GemmArgs& a) {
    if (a.m <= 0) return hipSuccess;
    if (!a.ap || !a.wp || !gemm_pk_supported(epi, a.m, a.n, a.k) || (epi == EPI_GLU && !a.wp2))
        return hipErrorInvalidValue;
    const dim3 block(256);
    const QkvRopeArgs f{};
    if (epi == EPI_GLU) {
        TL_KLAUNCH(gemm_pk_glu_kernel<1>, dim3(a.n / 32, (a.m + 127) / 128), block, pk_glu_lds_bytes(1), s, a);
        return hipGetLastError();
    }
    const bool res = epi == EPI_DEQUANT_RES;
    if (pk_split_narrow(a.m, a.n)) {
        const dim3 grid(a.n / 160, (a.m + 31) / 32);
        if (res) TL_KLAUNCH((gemm_pk_split_kernel<1, 5, EPI_DEQUANT_RES>), grid, block, pk_split_lds_bytes(1, 5), s, a, f);
        else TL_KLAUNCH((gemm_pk_split_kernel<1, 5, EPI_DEQUANT>), grid, block, pk_split_lds_bytes(1, 5), s, a, f);
    } else {
        const dim3 grid(a.n / 64, (a.m + 63) / 64);
        if (res) TL_KLAUNCH((gemm_pk_split_kernel<2, 2, EPI_DEQUANT_RES>), grid, block, pk_split_lds_bytes(2, 2), s, a, f);
        else TL_KLAUNCH((gemm_pk_split_kernel<2, 2, EPI_DEQUANT>), grid, block, pk_split_lds_bytes(2, 2), s, a, f);
    }
    return hipGetLastError();
}

hipError_t launch_gemm_pk_qkv(hipStream_t s, const GemmArgs& a, const QkvRopeArgs& f) {
    if (a.m <= 0) return hipSuccess;
    const int D = f.n_heads * kHeadDim, KVD = f.n_kv * kHeadDim;
    if (!a.ap || !a.wp || !f.q_out || !f.q_max || f.n_heads <= 0 || f.n_kv <= 0 || a.n != D + 2 * KVD ||
        a.k % 512 || a.n % 64)
        return hipErrorInvalidValue;
    TL_KLAUNCH((gemm_pk_split_kernel<2, 2, EPI_QKV_ROPE>), dim3(a.n / 64, (a.m + 63) / 64), dim3(256),
               pk_split_lds_bytes(2, 2), s, a, f);
    return hipGetLastError();
}

hipError_t init_gemm_pk_kernels() {
    const void* fns[] = {(const void*)gemm_pk_split_kernel<1, 5, EPI_DEQUANT>,
                         (const void*)gemm_pk_split_kernel<1, 5, EPI_DEQUANT_RES>,
                         (const void*)gemm_pk_split_kernel<2, 2, EPI_DEQUANT>,
                         (const void*)gemm_pk_split_kernel<2, 2, EPI_DEQUANT_RES>, (const void*)gemm_pk_glu_kernel<1>,
                         (const void*)gemm_pk_split_kernel<2, 2, EPI_QKV_ROPE>};
    const size_t bytes[] = {pk_split_lds_bytes(1, 5), pk_split_lds_bytes(1, 5), pk_split_lds_bytes(2, 2),
                            pk_split_lds_bytes(2, 2), pk_glu_lds_bytes(1), pk_split_lds_bytes(2, 2)};
    for (int i = 0; i < 6; i++) {
        const hipError_t e = hipFuncSetAttribute(fns[i], hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes[i]);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace tl
