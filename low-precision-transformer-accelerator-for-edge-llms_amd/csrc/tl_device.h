// tl_device.h -- device-side arithmetic shared by every kernel file.  Each
// helper is the exact operation sequence the CPU oracle (oracle/tl_oracle.c)
// performs, so kernels built from them agree with it bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "tl_internal.h"

namespace tl {

#define TL_DEV __device__ __forceinline__

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// scalar helpers
// ---------------------------------------------------------------------------

// exp(x): Cody-Waite reduction x = k ln2 + r (ln2 = 355/512 + remainder),
// degree-7 Taylor polynomial (1/n! in float32) in Horner form with explicit
// fused multiply-adds, times 2^k from the exponent field.  x < -80 -> 0.
TL_DEV float tl_expf(float x) {
    if (!(x >= -80.0f)) return 0.0f;
    if (x > 80.0f) x = 80.0f;
    const float log2e = 0x1.715476p+0f;
    const float c1 = 0x1.63p-1f;
    const float c2 = -0x1.bd0106p-13f;
    float kf = __builtin_rintf(x * log2e);
    float r = __builtin_fmaf(-kf, c1, x);
    r = __builtin_fmaf(-kf, c2, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    int k = (int)kf;
    return p * __int_as_float((k + 127) << 23);
}

// tl_expf without branches, the same value for every input: the argument is
// clamped to [-80, 80] before the reduction and the result is 0 below -80
// (and for NaN), as in tl_expf
TL_DEV float tl_expf_sel(float x) {
    const float xc = fminf(fmaxf(x, -80.0f), 80.0f);
    const float log2e = 0x1.715476p+0f;
    const float c1 = 0x1.63p-1f;
    const float c2 = -0x1.bd0106p-13f;
    float kf = __builtin_rintf(xc * log2e);
    float r = __builtin_fmaf(-kf, c1, xc);
    r = __builtin_fmaf(-kf, c2, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int k = (int)kf;
    const float e = p * __int_as_float((k + 127) << 23);
    return x >= -80.0f ? e : 0.0f;
}

// tl_expf for x <= 0 (a softmax argument: a score minus its row's maximum),
// the same value in fewer instructions: such x never reach the upper clamp;
// below -80 the select returns 0 whatever the reduction gave, so the lower
// clamp is not needed either; and from -80 to 0, k = rint(x log2e) lies in
// [-116, 0], where p 2^k is a normal float, so ldexp(p, k) equals the
// product with 2^k exactly.
TL_DEV float tl_expf_nonpos(float x) {
    const float log2e = 0x1.715476p+0f;
    const float c1 = 0x1.63p-1f;
    const float c2 = -0x1.bd0106p-13f;
    const float kf = __builtin_rintf(x * log2e);
    float r = __builtin_fmaf(-kf, c1, x);
    r = __builtin_fmaf(-kf, c2, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const float e = __builtin_amdgcn_ldexpf(p, (int)kf);
    return x >= -80.0f ? e : 0.0f;
}

// SiLU, TL:159-161: x / (1 + exp(-clip(x, -60, 60)))
TL_DEV float tl_silu(float x) {
    float c = x < -60.0f ? -60.0f : (x > 60.0f ? 60.0f : x);
    return __fdiv_rn(x, 1.0f + tl_expf(-c));
}

TL_DEV int8_t sat_i8(float v) {
    v = v > 127.0f ? 127.0f : v;
    v = v < -127.0f ? -127.0f : v;
    return (int8_t)(int)v;
}

// a / b rounded to nearest for many a over one b.  y = RN(1/b) is formed
// once; each quotient starts from q0 = RN(a y) and takes two residual
// corrections q <- RN(q + RN(a - b q) y), both fused multiply-adds.  The
// first leaves q within half an ulp plus 2^-46 relative of a / b (so
// faithful); the second is Markstein's correction, which from a faithful q
// and y within half an ulp of 1/b gives RN(a / b) exactly.  The proof needs
// normal residuals: callers take this path only when RnDiv::fast (set by
// rn_div_prep for |b| in [2^-64, 2^64]) and |a y| stays finite, and a
// correctly rounded division otherwise.  A quotient below the normal range may differ in its
// last bits; it rounds to integer 0 either way.
struct RnDiv {
    float b, y;
    bool fast;   // the same in every lane
};

TL_DEV RnDiv rn_div_prep(float b) {
    RnDiv d;
    d.b = b;
    d.y = __fdiv_rn(1.0f, b);
    const float ab = fabsf(b);
    d.fast = __builtin_amdgcn_readfirstlane((int)(ab >= 0x1p-64f && ab <= 0x1p64f)) != 0;
    return d;
}

TL_DEV float rn_div_fast(float a, const RnDiv& d) {
    const float q0 = a * d.y;
    const float q1 = __builtin_fmaf(__builtin_fmaf(-d.b, q0, a), d.y, q0);
    return __builtin_fmaf(__builtin_fmaf(-d.b, q1, a), d.y, q1);
}

// four quotients -> four saturated INT8 bytes (GI:39-41), x in byte 0
template <bool FAST>
TL_DEV unsigned quant4(float4 v, const RnDiv& d) {
    const float q0 = FAST ? rn_div_fast(v.x, d) : __fdiv_rn(v.x, d.b);
    const float q1 = FAST ? rn_div_fast(v.y, d) : __fdiv_rn(v.y, d.b);
    const float q2 = FAST ? rn_div_fast(v.z, d) : __fdiv_rn(v.z, d.b);
    const float q3 = FAST ? rn_div_fast(v.w, d) : __fdiv_rn(v.w, d.b);
    const unsigned b0 = (uint8_t)sat_i8(__builtin_rintf(q0));
    const unsigned b1 = (uint8_t)sat_i8(__builtin_rintf(q1));
    const unsigned b2 = (uint8_t)sat_i8(__builtin_rintf(q2));
    const unsigned b3 = (uint8_t)sat_i8(__builtin_rintf(q3));
    return b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
}

// GI:36-42 scale: max|x| / 127 in float64, 1.0 for an all-zero tensor
TL_DEV double quant_scale(float mx) { return mx != 0.0f ? (double)mx / 127.0 : 1.0; }

// GI:45-46 dequantization multiplier, formed in float64, rounded once
TL_DEV float deq_mult(double sx, float sw) { return (float)(sx * (double)sw); }

// 64-bit argmax key: order-preserving float bits above, (~index) below, so the
// maximum key is the largest logit with the lowest index (B4 tie-break).
TL_DEV unsigned long long argmax_key(float v, int32_t idx) {
    if (v == 0.0f) v = 0.0f;  // -0 and +0 compare equal in np.argmax
    unsigned u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xFFFFFFFFu - (unsigned)idx);
}

TL_DEV float key_logit(unsigned long long key) {
    unsigned u = (unsigned)(key >> 32);
    u = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
    return __uint_as_float(u);
}

TL_DEV int32_t key_index(unsigned long long key) {
    return (int32_t)(0xFFFFFFFFu - (unsigned)(key & 0xFFFFFFFFull));
}

// ---------------------------------------------------------------------------
// cross-lane exchange without the LDS crossbar (a ds_bpermute costs an LDS
// round trip per step): DPP moves inside rows of 16 lanes, gfx950's
// v_permlane16_swap / v_permlane32_swap across rows and wavefront halves.
// Every helper expects the whole wavefront active.
// ---------------------------------------------------------------------------
TL_DEV int lane_id() { return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// The wavefront's index in its workgroup as a wavefront-uniform (scalar)
// value, for every kernel that issues MFMAs.  MFMA instructions ignore EXEC:
// with no lane active, or some, an MFMA still multiplies and writes its whole
// accumulator.  A condition the compiler takes for lane-divergent (anything
// computed from threadIdx.x) becomes an EXEC mask, and the compiler drops the
// branch that skips a masked block when the block is short and holds no memory
// wait (it counts a masked-off instruction as a no-op), so an MFMA guarded by
// such a condition can run anyway and add a product that was meant to be
// skipped.  Conditions built from wave_id() and kernel arguments are uniform:
// they compile to scalar branches, which skip the MFMA for real.
TL_DEV int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// DPP controls
constexpr int kDppXor1 = 0xB1;          // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;          // quad_perm [2,3,0,1]
// row_ror:n hands lane j the value of lane (j - n) mod 16 of its row
constexpr int kDppRor4 = 0x124;         // row_ror:4  (lane - 4 within the row)
constexpr int kDppRor8 = 0x128;         // row_ror:8  (= lane ^ 8)
constexpr int kDppRor12 = 0x12C;        // row_ror:12 (lane + 4 within the row)
constexpr int kDppRowMirror = 0x140;    // lane 15 - j within the row
constexpr int kDppHalfMirror = 0x141;   // lane 7 - j within each half-row

// every control used reads a lane of the same row, so no lane takes the
// 0 given for out-of-row sources; the 0 lets the move fold into its user
template <int CTRL>
TL_DEV int dpp(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// the value of lane (lane ^ OFF): __shfl_xor(v, OFF) of a full wavefront
template <int OFF>
TL_DEV int lane_xor(int v) {
    static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8 || OFF == 16 || OFF == 32, "lane_xor: 1 .. 32");
    if constexpr (OFF == 1) {
        return dpp<kDppXor1>(v);
    } else if constexpr (OFF == 2) {
        return dpp<kDppXor2>(v);
    } else if constexpr (OFF == 4) {
        const int up = dpp<kDppRor12>(v), dn = dpp<kDppRor4>(v);
        return (lane_id() & 4) ? dn : up;
    } else if constexpr (OFF == 8) {
        return dpp<kDppRor8>(v);
    } else if constexpr (OFF == 16) {
        // rows 1, 3 of the first operand trade places with rows 0, 2 of the
        // second: p[0] = rows (0, 0, 2, 2), p[1] = rows (1, 1, 3, 3)
        const auto p = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
        return (int)((lane_id() & 16) ? p[0] : p[1]);
    } else {
        // the upper half of the first operand trades places with the lower
        // half of the second: p[0] = halves (lo, lo), p[1] = halves (hi, hi)
        const auto p = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
        return (int)((lane_id() & 32) ? p[0] : p[1]);
    }
}

template <int OFF>
TL_DEV float lane_xor(float v) {
    return __int_as_float(lane_xor<OFF>(__float_as_int(v)));
}

// lane ^ off for a wavefront-uniform run-time off (a power of two below 64)
TL_DEV float lane_xor_rt(float v, int off) {
    switch (off) {
        case 1: return lane_xor<1>(v);
        case 2: return lane_xor<2>(v);
        case 4: return lane_xor<4>(v);
        case 8: return lane_xor<8>(v);
        case 16: return lane_xor<16>(v);
        default: return lane_xor<32>(v);
    }
}

// pair sums of the xor-16 / xor-32 levels of a butterfly: both swap results
// added give v[lane] + v[lane ^ OFF] in every lane
template <int OFF>
TL_DEV float pair_sum(float v) {
    static_assert(OFF == 16 || OFF == 32, "pair_sum: 16 or 32");
    const unsigned u = __float_as_uint(v);
    const auto p = OFF == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                             : __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// the four row values of a row-uniform register, combined by the caller
TL_DEV int row_value(int v, int row) { return __builtin_amdgcn_readlane(v, 16 * row); }

// integer sum over the wavefront (exact in any order), in every lane
TL_DEV int wave_sum_i32(int v) {
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    v += dpp<kDppHalfMirror>(v);
    v += dpp<kDppRowMirror>(v);   // every lane: its row's sum
    return (row_value(v, 0) + row_value(v, 1)) + (row_value(v, 2) + row_value(v, 3));
}

// maximum over the wavefront (order-free), in every lane
TL_DEV float wave_max_f32(float v) {
    v = fmaxf(v, __int_as_float(dpp<kDppXor1>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp<kDppXor2>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp<kDppHalfMirror>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp<kDppRowMirror>(__float_as_int(v))));
    const int iv = __float_as_int(v);
    return fmaxf(fmaxf(__int_as_float(row_value(iv, 0)), __int_as_float(row_value(iv, 1))),
                 fmaxf(__int_as_float(row_value(iv, 2)), __int_as_float(row_value(iv, 3))));
}

// maximum over each half-wavefront (lanes 0-31, 32-63), in every lane of it
TL_DEV float half_max_f32(float v) {
    v = fmaxf(v, __int_as_float(dpp<kDppXor1>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp<kDppXor2>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp<kDppHalfMirror>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp<kDppRowMirror>(__float_as_int(v))));
    const unsigned u = __float_as_uint(v);
    const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

// the fixed 64-wide butterfly: levels 32, 16, 8, 4, 2, 1, each adding lane
// pairs (lane, lane ^ off) (same tree as or_block_sum64)
TL_DEV float wave_butterfly_sum(float v) {
    v = pair_sum<32>(v);
    v = pair_sum<16>(v);
    v = v + lane_xor<8>(v);
    v = v + lane_xor<4>(v);
    v = v + lane_xor<2>(v);
    v = v + lane_xor<1>(v);
    return v;
}

// the same butterfly over each half-wavefront: levels 16, 8, 4, 2, 1
TL_DEV float half_butterfly_sum(float v) {
    v = pair_sum<16>(v);
    v = v + lane_xor<8>(v);
    v = v + lane_xor<4>(v);
    v = v + lane_xor<2>(v);
    v = v + lane_xor<1>(v);
    return v;
}

TL_DEV unsigned long long max_u64(unsigned long long a, unsigned long long b) { return b > a ? b : a; }

template <int CTRL>
TL_DEV unsigned long long dpp_u64(unsigned long long v) {
    const unsigned lo = (unsigned)dpp<CTRL>((int)(unsigned)(v & 0xFFFFFFFFull));
    const unsigned hi = (unsigned)dpp<CTRL>((int)(unsigned)(v >> 32));
    return ((unsigned long long)hi << 32) | lo;
}

TL_DEV unsigned long long row_max_u64(unsigned long long v) {
    v = max_u64(v, dpp_u64<kDppXor1>(v));
    v = max_u64(v, dpp_u64<kDppXor2>(v));
    v = max_u64(v, dpp_u64<kDppHalfMirror>(v));
    return max_u64(v, dpp_u64<kDppRowMirror>(v));
}

TL_DEV unsigned long long row_value_u64(unsigned long long v, int row) {
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(v & 0xFFFFFFFFull), 16 * row);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(v >> 32), 16 * row);
    return ((unsigned long long)hi << 32) | lo;
}

// Decode-timeline stamps: with ts set, lane 0 of the wavefront stores the
// GPU clock (wall_clock64, constant rate) read when the kernel reached this
// object and when the object leaves scope (on every return path) at
// ts[2 * wave_id] and ts[2 * wave_id + 1].  Without ts it does nothing.
struct WaveStamp {
    unsigned long long* p;
    unsigned long long t0;
    TL_DEV WaveStamp(unsigned long long* ts, int64_t wave_id) : p(nullptr), t0(0) {
        if (ts != nullptr) {
            t0 = wall_clock64();
            if ((threadIdx.x & 63) == 0) p = ts + 2 * wave_id;
        }
    }
    TL_DEV ~WaveStamp() {
        if (p != nullptr) {
            const unsigned long long t1 = wall_clock64();
            p[0] = t0;
            p[1] = t1;
        }
    }
};

// maximum of 64-bit keys over the wavefront, in every lane
TL_DEV unsigned long long wave_max_u64(unsigned long long v) {
    v = row_max_u64(v);
    return max_u64(max_u64(row_value_u64(v, 0), row_value_u64(v, 1)),
                   max_u64(row_value_u64(v, 2), row_value_u64(v, 3)));
}

// maximum of 64-bit keys over each half-wavefront, in every lane of it
TL_DEV unsigned long long half_max_u64(unsigned long long v) {
    v = row_max_u64(v);
    const unsigned lo = (unsigned)(v & 0xFFFFFFFFull), hi = (unsigned)(v >> 32);
    const auto pl = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto ph = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    return max_u64(((unsigned long long)ph[0] << 32) | pl[0], ((unsigned long long)ph[1] << 32) | pl[1]);
}

// 128-bit loads that stay 128-bit: weights stream through once (non-temporal)
TL_DEV v4i ld_nt16(const int8_t* p) { return __builtin_nontemporal_load((const v4i*)p); }
TL_DEV v4i ld16(const int8_t* p) { return *(const v4i*)p; }

TL_DEV int sdot4v(v4i a, v4i b, int acc) {
    acc = __builtin_amdgcn_sdot4(a[0], b[0], acc, false);
    acc = __builtin_amdgcn_sdot4(a[1], b[1], acc, false);
    acc = __builtin_amdgcn_sdot4(a[2], b[2], acc, false);
    acc = __builtin_amdgcn_sdot4(a[3], b[3], acc, false);
    return acc;
}

TL_DEV int sdot4x4(int4 a, int4 b, int acc) {
    acc = __builtin_amdgcn_sdot4(a.x, b.x, acc, false);
    acc = __builtin_amdgcn_sdot4(a.y, b.y, acc, false);
    acc = __builtin_amdgcn_sdot4(a.z, b.z, acc, false);
    acc = __builtin_amdgcn_sdot4(a.w, b.w, acc, false);
    return acc;
}

// v[0] + v[1] + ... + v[n-1] added in index order, starting from 0 (the
// softmax denominator over block sums); up to 32 values are read before the
// first add, so the chain costs one LDS latency instead of n
TL_DEV float ordered_sum(const float* v, int n) {
    float t = 0.0f;
    if (n <= 32) {
        float r[32];
#pragma unroll
        for (int i = 0; i < 32; i++) r[i] = v[i < n ? i : 0];
#pragma unroll
        for (int i = 0; i < 32; i++)
            if (i < n) t = t + r[i];
        return t;
    }
    for (int i = 0; i < n; i++) t = t + v[i];
    return t;
}

// ordered_sum for 16-byte aligned v whose allocation holds 3 readable floats
// past v[n - 1]: n <= 8 values come in one or two 16-byte reads
TL_DEV float ordered_sum_aligned(const float* v, int n) {
    if (n > 8) return ordered_sum(v, n);
    const float4 a = *(const float4*)v;
    const float4 b = n > 4 ? *(const float4*)(v + 4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float r[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++)
        if (i < n) t = t + r[i];
    return t;
}

// block-wide max of a non-negative float (all threads get the result)
TL_DEV float block_max(float v, float* red /* >= 16 floats */) {
    v = wave_max_f32(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
    for (int i = 1; i < nw; i++) m = fmaxf(m, red[i]);
    return m;
}

// NumPy pairwise sum of sq[0 .. plan.leaf_len*plan.n_leaves) (a perfect
// tree): 8 strided accumulators per leaf, ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7))
// per leaf, then leaves combined pairwise level by level.  scr needs
// 10 * n_leaves floats.  Returns the sum in every thread.
TL_DEV float block_pairwise_sum(const float* sq, PwPlan plan, float* scr) {
    const int tid = threadIdx.x, nt = blockDim.x;
    const int L = plan.n_leaves, len = plan.leaf_len;
    float* part = scr;           // [8 L]
    float* lv0 = scr + 8 * L;    // [L]
    float* lv1 = lv0 + L;        // [L]
    for (int idx = tid; idx < 8 * L; idx += nt) {
        // leaf_len <= 128: at most 16 steps, read before the in-order sum
        const float* a = sq + (idx >> 3) * len + (idx & 7);
        float v[16];
#pragma unroll
        for (int t = 0; t < 16; t++) v[t] = a[min(8 * t, len - 8)];
        float r = v[0];
#pragma unroll
        for (int t = 1; t < 16; t++)
            if (8 * t < len) r = r + v[t];
        part[idx] = r;
    }
    __syncthreads();
    for (int leaf = tid; leaf < L; leaf += nt) {
        const float* r = part + 8 * leaf;
        lv0[leaf] = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    }
    __syncthreads();
    float* cur = lv0;
    float* nxt = lv1;
    for (int w = L; w > 1; w >>= 1) {
        for (int i = tid; i < (w >> 1); i += nt) nxt[i] = cur[2 * i] + cur[2 * i + 1];
        __syncthreads();
        float* t = cur; cur = nxt; nxt = t;
    }
    return cur[0];
}

}  // namespace tl
