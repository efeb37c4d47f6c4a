// tl_internal.h -- declarations shared by the HIP kernels (tl_kernels.hip) and
// the C++ runtime (tl_runtime.hip).  Not part of the public C-ABI.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tl {

// Perfect pairwise-summation tree for a row width n: NumPy's float32 reduction
// splits n in halves down to leaves of <= 128 elements, each leaf summed with
// eight strided accumulators.  Widths supported on the device are those whose
// halving chain stays on multiples of eight (2048 = 16 x 128, 5632 = 64 x 88).
struct PwPlan {
    int32_t leaf_len;   // elements per leaf, multiple of 8, <= 128
    int32_t n_leaves;   // power of two
};
bool make_pw_plan(int32_t n, PwPlan* plan);

// KV cache geometry.  One plane per (sequence, layer, kv head) holds max_pos
// tokens of head_dim = 64 int8 values, laid out for coalesced reads:
//   K plane: [max_pos/64 blocks][4 dim-groups of 16][64 tokens][16 bytes]
//            so a wavefront whose lane t reads token t of a block issues four
//            fully coalesced 1 KiB loads;
//   V plane: [max_pos/16 groups][64 dims][16 tokens]
//            so lane d reading dimension d of 16 consecutive tokens issues one
//            fully coalesced 1 KiB load.
constexpr int kHeadDim = 64;
struct KvGeom {
    int8_t* k;           // base of all K planes
    int8_t* v;           // base of all V planes
    int32_t n_layers;
    int32_t n_kv_heads;
    int32_t max_pos;
    __host__ __device__ int64_t plane(int32_t seq, int32_t layer, int32_t g) const {
        return (((int64_t)seq * n_layers + layer) * n_kv_heads + g) * (int64_t)max_pos * kHeadDim;
    }
    __host__ __device__ static int64_t k_off(int32_t t, int32_t d) {
        return (int64_t)(t >> 6) * 4096 + (d >> 4) * 1024 + (t & 63) * 16 + (d & 15);
    }
    __host__ __device__ static int64_t v_off(int32_t t, int32_t d) {
        return (int64_t)(t >> 4) * 1024 + d * 16 + (t & 15);
    }
};

// Per-row description used by the row-parallel kernels (prefill rows of one
// sequence, or one row per sequence in batched decode).
struct RowMap {
    const int32_t* seq;  // [rows] sequence (KV plane) of each row
    const int32_t* pos;  // [rows] position of each row
};

enum GemvEpi : int {
    EPI_DEQUANT = 0,      // y = f32(acc) * f32(sx * sw[n])
    EPI_DEQUANT_RES = 1,  // y = residual + f32(acc) * f32(sx * sw[n])
    EPI_REQUANT = 2,      // y8 = sat(rne(f32(acc) * m[n]))
    EPI_GLU = 3,          // y = silu(gate) * up, both dequantized
    EPI_ARGMAX = 4,       // argmax of dequantized logits into a 64-bit key
    EPI_RAW = 5,          // acc only
    EPI_ACC = 6,          // acc[m][n] += the K slice's sum (integer atomic add; the row prologue that
                          // follows folds the sums and clears them)
    EPI_QKV_ROPE = 7,     // prefill Q|K|V: dequantize, RoPE on Q and K, K / V quantized into the cache,
                          // rotated Q out in float32 with its row maximum (launch_gemm_pk_qkv)
    EPI_ACC_F32 = 8,      // EPI_ACC with a float32 A that gemm_rows32 quantizes itself (GemmArgs::af)
};

// activation prologue of the fused decode GEMV
enum GemvPro : int {
    PRO_X8 = 0,       // x is already INT8 with its scale
    PRO_QUANT = 1,    // x float32 -> per-tensor INT8 (GI:36-42)
    PRO_RMSNORM = 2,  // x float32 -> RMSNorm (TL:45-50) -> INT8
};

constexpr int kMaxGroupHeads = 8;

struct GemvArgs {
    const float* xf;         // [K] float32 activation (fused prologues)
    const float* gamma;      // [K] RMSNorm gain (PRO_RMSNORM)
    float eps;
    PwPlan plan;
    const int8_t* w;         // [N][K]
    const int8_t* w2;        // [N][K] up weights (EPI_GLU)
    const float* ws;         // [N] weight scales or requant multipliers
    const float* ws2;        // [N] up-weight scales (EPI_GLU)
    const int8_t* x;         // [K] (row stride x_stride for multi-row)
    const double* xs;        // [1] activation scale (per row)
    const float* residual;   // [N]
    float* y;                // [N]
    int8_t* y8;              // [N] (EPI_REQUANT)
    int32_t* acc;            // [N] optional raw accumulators
    unsigned long long* key; // argmax slot (EPI_ARGMAX)
    unsigned long long* wg_keys; // EPI_ARGMAX: one key per workgroup (no atomic) instead of key
    int32_t n, k;
    unsigned long long* ts;  // decode timeline: [waves][2] clock stamps, or null
};

struct GemmArgs {
    const int8_t* a;          // [M][K]
    const int8_t* w;          // [N][K]
    const int8_t* w2;         // [N][K] up weights (GLU)
    const double* as;         // [M] row scales
    const float* ws;          // [N]
    const float* ws2;         // [N]
    const float* residual;    // [M][N]
    float* y;                 // [M][N]
    int32_t* acc;             // [M][N] raw (EPI_RAW) or [splits][M][N] partials
    int32_t m, n, k;
    int32_t k_split;          // K elements per split (multiple of 64; gemm_rows32: multiple of 32, 0 = K)
    const int8_t* wp;         // packed copy of w (MFMA operand blocks, pack_weights_kernel) or null
    const int8_t* wp2;        // packed copy of w2
    unsigned long long* key;  // EPI_ARGMAX: [N / 32 tiles][M] best key of each tile and row
    const int8_t* ap;         // A in MFMA operand blocks (rows padded to gemm_pk_row_pad()) for
                              // launch_gemm_pk, or null
    // gemm_rows32 EPI_ACC_F32 only: A is the float32 [M][K] row-major
    // matrix quantized per row here (quantize_int8, GI:36-42) at the maximum
    // of the amax_n (a multiple of 4, at most 32) values amax[row][..], the
    // row's parts' max |x|; the row scales go to as_out (a and as unused)
    const float* af;
    const float* amax;
    int32_t amax_n;
    double* as_out;
};

// Weight tiles to bring into L2 ahead of the GEMM that reads them, by extra
// workgroups of a row kernel launched before it.  Workgroups go to the 8 XCDs
// round-robin by linear id, and the GEMMs that take a prefetch place the
// workgroups of column tile t on XCD t % 8 (their grids have a multiple of 8
// column tiles in x), so the workgroups added on XCD x load tiles x, x + 8,
// ... of every matrix: the GEMM then reads them from its own XCD's L2.
struct L2Prefetch {
    const int8_t* w[2];    // the packed weight copies (nmat), or w[0] null: none
    int32_t nmat;
    int32_t ntiles;        // column tiles, a multiple of 8
    int64_t tile_bytes;    // contiguous bytes of one tile (all of its K blocks), a multiple of 16
    int32_t* sink;         // a word the loads' combined value is written to, never in practice
};

// ---- launchers (tl_kernels.hip) ------------------------------------------
// packed: q is written in the packed GEMM operand layout (launch_gemm_pk)
// instead of row-major; needs n % 64 == 0 and n <= 6144 (else invalid value)
hipError_t launch_rmsnorm_quant(hipStream_t s, const float* x, const float* g, int32_t rows,
                                int32_t n, float eps, PwPlan plan, float* y, int8_t* q,
                                double* scales, bool packed = false, const L2Prefetch* pf = nullptr);
// zero: optional [rows][zero_n] int32 buffer (zero_n % 4 == 0, 16-byte
// aligned) each row's workgroup clears after quantizing
hipError_t launch_quantize_rows(hipStream_t s, const float* x, int32_t rows, int32_t n,
                                int8_t* q, double* scales, int32_t* zero = nullptr, int32_t zero_n = 0,
                                bool packed = false, const L2Prefetch* pf = nullptr);

// RMSNorm row prologue that first finishes a K-sliced small-M GEMM with a
// residual epilogue: its integer sums acc (EPI_ACC, rows x n) are dequantized
// with the GEMM's A-row scales and weight scales exactly as that GEMM's
// DEQUANT_RES epilogue would (x += f32(acc) f32(sx sw), x written back),
// cleared to zero for the next GEMM, and the row then goes through RMSNorm
// and quantization into q / scales
struct FoldArgs {
    float* x;             // [rows][n] residual, overwritten with the sum
    int32_t* acc;         // [rows][n]
    const double* as;     // [rows] the GEMM's A-row scales (may alias scales: read first)
    const float* ws;      // [n]
    const float* g;       // [n] RMSNorm gains
    int32_t rows, n;
    float eps;
    PwPlan plan;
    int8_t* q;            // [rows][n]
    double* scales;       // [rows]
    int32_t* zero;        // or null: [rows][zero_n] int32 the kernel also clears (consumed integer sums)
    int32_t zero_n;
    L2Prefetch pf;        // the next GEMM's weight tiles (pf.w[0] null: none)
};
hipError_t launch_rows_fold(hipStream_t s, const FoldArgs& f);
hipError_t launch_quantize_tensor(hipStream_t s, const float* x, int64_t n, int8_t* q,
                                  double* scale, float* scratch_max);
hipError_t launch_quantize_weight_rows(hipStream_t s, const float* w, int32_t rows, int32_t n,
                                       int8_t* q, float* scales);
hipError_t launch_gemv(hipStream_t s, int epi, const GemvArgs& a);
constexpr int kSkinnyTiles = 4096;     // output tiles of 32 columns the split small-M GEMM counts
constexpr int kSkinnyMaxSlices = 8;   // K slices of the small-M GEMM (LDS holds the other 7 partial tiles)
hipError_t launch_gemm_rows32(hipStream_t s, int epi, const GemmArgs& a, int32_t waves = 16);
hipError_t launch_pack_weights(hipStream_t s, const int8_t* w, int32_t n, int32_t k, int8_t* wp);

hipError_t launch_gemm_skinny(hipStream_t s, int epi, const GemmArgs& a, int32_t slices, int32_t* part,
                              unsigned* counters);
hipError_t launch_gemm(hipStream_t s, int epi, const GemmArgs& a, int32_t splits);
hipError_t launch_gemm_reduce(hipStream_t s, int epi, const GemmArgs& a, int32_t splits);
hipError_t launch_qkv_post(hipStream_t s, const float* qkv, int32_t rows, int32_t n_heads,
                           int32_t n_kv_heads, RowMap rm, const float* cos, const float* sin,
                           KvGeom kv, int32_t layer, const float* kv_sk, const float* kv_sv,
                           int8_t* q8, double* q_scale, float* q_rot_out, bool append_kv = true);
constexpr int kTileMaxKeys = 4096;   // context limit of launch_attention_tiles (LDS)
// qf / qmax (optional, instead of q8 / q_scale): rotated Q rows in float32
// ([rows][D]) and their maxima max|q| as float bits ([rows][kQmaxStride],
// element 0),
// quantized by the kernel exactly as qkv_post quantizes them
hipError_t launch_attention_tiles(hipStream_t s, const int8_t* q8, const double* q_scale, int32_t rows,
                                  int32_t n_heads, int32_t n_kv_heads, int32_t seq, int32_t pos0, KvGeom kv,
                                  int32_t layer, const float* kv_sk, const float* kv_sv, float* out,
                                  const float* qf = nullptr, const unsigned* qmax = nullptr);
// Optional debug outputs of row 0 (the decode-step capture): INT32 scores and
// INT8 probabilities of keys key0 .. key0 + n_keys - 1 per query head
// ([n_heads][n_keys]) and the f32 score scale per query head.
struct AttnDebug {
    int32_t* scores = nullptr;
    int8_t* probs = nullptr;
    float* score_scale = nullptr;
    int32_t key0 = 0;
    int32_t n_keys = 0;
};
hipError_t launch_attention(hipStream_t s, const int8_t* q8, const double* q_scale, int32_t rows,
                            int32_t n_heads, int32_t n_kv_heads, RowMap rm, KvGeom kv,
                            int32_t layer, const float* kv_sk, const float* kv_sv, float* out,
                            int32_t max_t, AttnDebug dbg = AttnDebug());
// float32 model of the analysis report (tl_float.hip)
hipError_t launch_linear_f32(hipStream_t s, const float* x, const float* w, const float* b, const float* residual,
                             int32_t m, int32_t n, int32_t k, float* y);
hipError_t launch_attention_f32(hipStream_t s, const float* q, const float* k, const float* v, int32_t seq,
                                int32_t n_heads, int32_t n_kv, float scale, float* out, float* scores,
                                float* weights);
hipError_t launch_rope(hipStream_t s, float* v, int32_t rows, int32_t n_heads, const int32_t* pos,
                       const float* cos, const float* sin);
hipError_t launch_softmax_rows(hipStream_t s, const float* x, int32_t rows, int32_t n, float* p);
hipError_t launch_silu_mul(hipStream_t s, const float* g, const float* u, int64_t n, float* y);
hipError_t launch_dequant_i32(hipStream_t s, const int32_t* acc, int64_t n, int32_t cols, float m,
                              const float* bias, float* y);
hipError_t launch_embed(hipStream_t s, const int32_t* tokens, int32_t rows, int32_t d, int32_t vocab,
                        const int8_t* emb, const float* emb_s, float* x);
hipError_t launch_reset_keys(hipStream_t s, unsigned long long* keys, int32_t n);
// embedding of the next step's token (row 0), written by the finalize kernel
struct EmbedNext {
    const int8_t* emb;
    const float* emb_s;
    int32_t d, vocab;
    float* x;            // nullptr: no embedding
    int32_t* row_pos;
    // stop condition of the row's sequence (stop_condition_unit.sv:18-37):
    // after the token equal to *eos (< 0: none) is recorded, *stopped is set;
    // while it is set a step records nothing and re-embeds the same token at
    // the same position, so further replays leave the state as it is
    const int32_t* eos;  // nullptr: no stop check
    int32_t* stopped;    // 1 after EOS, 2 after a host abort
    // host abort (stop_condition_unit.sv:26-28, abort outranks EOS): a word
    // of pinned host memory the host sets; a step that reads it non-zero
    // records nothing and sets *stopped = 2.  *stop_host (pinned host
    // memory) mirrors *stopped for the host's per-step watch.  Null: no
    // abort check, no mirror.
    const int32_t* abort_word;
    int32_t* stop_host;
    unsigned long long* ts;   // decode timeline: [1][2] clock stamps, or null
};
hipError_t launch_finalize_tokens(hipStream_t s, unsigned long long* keys, int32_t rows,
                                  int32_t* token_cur, int32_t* tokens_out, int32_t out_stride,
                                  int32_t* n_gen, int32_t* cursor, float* best_logit, int32_t advance,
                                  const unsigned long long* wg_keys = nullptr, int32_t n_wg = 0,
                                  EmbedNext nx = EmbedNext{});
// workgroups launch_gemv_fused uses for this prologue / epilogue / shape
int32_t gemv_fused_workgroups(int pro, int epi, int32_t n, int32_t k);
int64_t gemv_fused_wavefronts(int pro, int epi, int32_t n, int32_t k);
hipError_t launch_argmax_rows(hipStream_t s, const float* logits, int32_t rows, int32_t n,
                              unsigned long long* keys);
hipError_t launch_argmax_tiles(hipStream_t s, const unsigned long long* part, int32_t tiles, int32_t rows,
                               unsigned long long* keys);
hipError_t init_kernels();
hipError_t init_decode_kernels();
hipError_t init_prefill_kernels();
hipError_t init_skinny_kernels();
hipError_t launch_fill_u32(hipStream_t s, unsigned* p, int32_t n, unsigned v);
hipError_t launch_causal_mask_i32(hipStream_t s, const int32_t* scores, int32_t rows, int32_t cols, int32_t qb,
                                  int32_t kb, int32_t qrc, int32_t kcc, int32_t* out);
hipError_t launch_rope_q16(hipStream_t s, const int8_t* x, int32_t rows, int32_t n_heads, const int32_t* pos,
                           const float* cosb, const float* sinb, int32_t n_pos, int8_t* out);
hipError_t launch_argmax_i32(hipStream_t s, const int32_t* v, int32_t n, unsigned long long* key);
hipError_t launch_requant_q16(hipStream_t s, const int32_t* acc, const uint32_t* scale, int32_t n, int32_t active,
                              int32_t lanes_per_scale, int32_t nonnegative_only, int8_t* y);

hipError_t launch_gemm32(hipStream_t s, int epi, const GemmArgs& a, bool tile);
// prefill GEMM on packed A (a.ap) and packed weights (a.wp, a.wp2): DEQUANT,
// DEQUANT_RES or GLU where gemm_pk_supported(); packed A holds row r's 16-byte
// piece p (K bytes [16 p, 16 p + 16)) at byte ((r / 32) (K / 32) + p / 2) 1024 +
// ((p % 2) 32 + r % 32) 16, rows padded to a multiple of gemm_pk_row_pad()
bool gemm_pk_supported(int epi, int32_t m, int32_t n, int32_t k);
// the prefill Q|K|V GEMM with qkv_post's work in its epilogue (EPI_QKV_ROPE):
// RoPE on Q and K at each row's position, K and V quantized with the static
// per-head scales into the cache, rotated Q written to q_out ([M][D] float32)
// and max|q| of each row folded into q_max[kQmaxStride row] (float bits,
// atomic max; zero beforehand).  Needs N = D + 2 KVD with D, KVD multiples
// of 64.  One 128-byte line per row: the 32 heads' atomics on a row then
// share a line with no other row's (4-byte rows took the GEMM from 13.5 to
// 15.5 us, 16-byte rows measured 13.3-13.7 us).
constexpr int kQmaxStride = 32;
struct QkvRopeArgs {
    const float* cosb;
    const float* sinb;
    RowMap rm;
    KvGeom kv;
    int32_t layer, n_heads, n_kv;
    const float* kv_sk;
    const float* kv_sv;
    float* q_out;
    unsigned* q_max;
};
hipError_t launch_gemm_pk_qkv(hipStream_t s, const GemmArgs& a, const QkvRopeArgs& f);
int32_t gemm_pk_row_pad();
hipError_t launch_gemm_pk(hipStream_t s, int epi, const GemmArgs& a);
hipError_t init_gemm_pk_kernels();
hipError_t launch_gemv_fused(hipStream_t s, int pro, int epi, const GemvArgs& a);
// Q|K|V rows as the integer sums of a K-sliced GEMM with its dequantization
// scales (batched decode; the grouped attention kernel only)
struct QkvSums {
    const int32_t* acc;   // [rows][D + 2 KVD]
    const double* as;     // [rows] A-row scales of the GEMM
    const float* ws;      // [D + 2 KVD] weight scales
};
// launch_attention_decode takes the grouped (many-row) kernel for these
// arguments; the only path that accepts QkvSums
bool attention_decode_grouped(int32_t rows, int32_t n_heads, int32_t n_kv, int32_t max_t);
// out_max (the grouped kernel only): [rows][n_heads] max |output| of each head
hipError_t launch_attention_decode(hipStream_t s, const float* qkv, int32_t rows, int32_t n_heads, int32_t n_kv,
                                   RowMap rm, const float* cos, const float* sin, KvGeom kv, int32_t layer,
                                   const float* kv_sk, const float* kv_sv, float* out, int32_t max_t,
                                   unsigned long long* ts = nullptr, const QkvSums* sums = nullptr,
                                   float* out_max = nullptr);
hipError_t launch_embed_step(hipStream_t s, const int32_t* tok_by_seq, const int32_t* seq_of_row, int32_t rows,
                             const int32_t* cursor, int32_t* row_pos, int32_t d, int32_t vocab, const int8_t* emb,
                             const float* emb_s, float* x);
hipError_t launch_step_rows(hipStream_t s, const int32_t* seq_of_row, int32_t rows,
                            const int32_t* cursor, int32_t* row_pos);
hipError_t launch_kv_scatter(hipStream_t s, KvGeom kv, int32_t seq, int32_t layer, int32_t g,
                             int32_t t0, int32_t n, const int8_t* k_rows, const int8_t* v_rows);
hipError_t launch_kv_gather(hipStream_t s, KvGeom kv, int32_t seq, int32_t layer, int32_t g,
                            int32_t t0, int32_t n, int8_t* k_rows, int8_t* v_rows);

// Kernel timing for the profiler.  While a profiled operation runs, its
// first kernel records `start` when that kernel starts and every kernel
// records `stop` when it ends: the dispatch's own timestamps, without queue or
// launch time, so the durations are those a kernel trace reports.
struct KernelTiming {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
    bool used = false;
};
KernelTiming& kernel_timing();   // this host thread's

#define TL_KLAUNCH(kernel, grid, block, lds, stream, ...)                                                   \
    do {                                                                                                   \
        ::tl::KernelTiming& kt_ = ::tl::kernel_timing();                                                   \
        if (kt_.stop) {                                                                                    \
            hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, kt_.used ? nullptr : kt_.start, kt_.stop, \
                                  0, __VA_ARGS__);                                                         \
            kt_.used = true;                                                                               \
        } else {                                                                                           \
            hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);                             \
        }                                                                                                  \
    } while (0)

}  // namespace tl
