// The int8 MFMA GEMM for many activation vectors (prefill, batched verify):
// y[m][n] = sum_b s_x[m,b] s_w[n,b] P_b[m][n]  (+ Q4: sum_b bias[n,b] s_x[m,b] sum_k q_x[m,32b+k]),
// P_b[m][n] = sum_k q_w[n,32b+k] q_x[m,32b+k], exact in int32.
//
// One v_mfma_i32_32x32x32_i8 is one nncpu block (K = 32) of a 32 x 32 tile,
// so its result is exactly the tile's block dots P_b. The A operand is the
// weights (rows n), B the activations (tokens m); lane l holds row / token
// l%32 and K-half l/32 (16 bytes). Result element (i, j) sits in lane
// j + 32h, register r, with i = (r/4)*8 + 4h + r%4: a lane owns one token
// and 16 weight rows of each 32 x 32 tile.
//
// Epilogue per block and output: acc = fma(f32(P), s_w * s_x, acc) in f32,
// P and the scale product being exact, with the f32 sum folded into an f64
// total every 8 blocks (an f32 sum over K = 18944 would take most of the
// 1e-5 tolerance next to nncpu's own f32 rounding; chunks of 8 keep the
// error within 8 f32 roundings of the absolute block terms). The scale
// products s_w[n] s_x[m] come from the matrix unit too: one
// v_mfma_f32_32x32x1_2b_f32 forms the outer products of two blocks exactly,
// already in the result layout, so each lane needs one scale per block
// instead of sixteen; and the Q4 bias term sum_b bias[n,b] (s_x sum q_x)[m,b]
// is an outer-product sum, one v_mfma_f32_32x32x2f32 per two blocks
// accumulating into the same f32 tile. nncpu's per-32 BF16 scales make this
// epilogue, not the int8 MFMA, the compute bound: 2 VALU ops per output and
// block (the int32 -> f32 conversion and the FMA) against 32 MACs.
//
// Workgroup: 128 weight rows x 128 tokens, 16 waves (4 per SIMD, to hide the
// MFMA -> VALU latency), each wave one 32 x 32 tile. The K loop runs over
// chunks of KB blocks through a ring of three LDS stages filled by direct
// global -> LDS loads (global_load_lds_dwordx4, no staging registers), so
// two chunks are in flight while one is computed. Scales come from
// block-major f32 copies (weights: built at upload; activations: written by
// the quantizer) so each stage's scales are contiguous 16-byte pieces too.
// Grids too small for the 256 CUs are split along K; the partial tiles go
// to a workspace in f64 and a second kernel adds them in split order.

#include "common.h"

namespace nnh {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

constexpr int TILE = 128;  // weight rows and tokens per workgroup
constexpr int GEMM_MAX_SPLITS = 8;
constexpr int NW = 16;     // waves per workgroup (4 per SIMD: latency hiding)
constexpr int WN = 4;      // waves along the rows: each wave owns TILE / WN rows ...
constexpr int WM = 4;      // ... and TILE / WM tokens
static_assert(WN * WM == NW && TILE == 32 * WN && TILE == 32 * WM, "one 32 x 32 tile per wave");

template <int DT, int KB>
struct GStage {
    static constexpr int QB = DT == 1 ? 32 : 16;  // weight bytes per row and block
    uint8_t A[KB * TILE * QB];                    // [blk][row][QB]
    int8_t B[KB * TILE * 32];                     // [blk][token][32]
    float SW[KB * TILE];                          // [blk][row]
    float SX[KB * TILE];                          // [blk][token]
    float BI[DT == 2 ? KB * TILE : 4];            // [blk][row]   (Q4)
    float SXQ[DT == 2 ? KB * TILE : 4];           // [blk][token] (Q4)
};

// Direct-load instructions per stage (64 lanes x 16 bytes each), dealt
// round-robin to the waves: wave w issues instructions w, w + NW, ...,
// PER_WAVE of them if w < I_TOTAL % NW (or the split is even), else one
// fewer.
template <int DT, int KB>
struct GPlan {
    static constexpr int I_A = KB * TILE * GStage<DT, KB>::QB / 16 / 64;
    static constexpr int I_B = KB * TILE * 32 / 16 / 64;
    static constexpr int I_S = KB * TILE * 4 / 16 / 64;  // one f32 [blk][TILE] table
    static constexpr int N_S = (DT == 2 ? 4 : 2) * I_S;
    static constexpr int I_TOTAL = I_A + I_B + N_S;
    static constexpr int PER_WAVE = (I_TOTAL + NW - 1) / NW;
    static_assert(KB * TILE * 4 % 1024 == 0, "scale tables must fill whole load instructions");
    static_assert(2 * PER_WAVE < 64, "vmcnt holds at most 63");
    __device__ static bool full(int wave) { return I_TOTAL % NW == 0 || wave < I_TOTAL % NW; }
};

struct GArgs {
    const uint8_t* qs;  // weights, nncpu row-major quants
    const float* swT;   // [nb][rows_pad] weight scales; Q4 biases follow at + nb * rows_pad
    const int8_t* aq;   // activation quants [n_tok][cols]
    const float* sxT;   // [nb][tok_pad] activation scales, then [nb][tok_pad] scale * sum(q)
    double* ws;         // split-K partial tiles [split][tile][wave][16][64] (splits > 1)
    int rows, rows_pad, nb, n_tok, tok_pad, mtiles, tiles, splits;
    int kb0, kb1;       // this workgroup's blocks [kb0, kb1)
    size_t qrow, cols;
};

// Issue this wave's share of the direct loads for chunk `chunk`. Rows,
// tokens and blocks past the end are clamped to the last valid one: they
// feed outputs that are never stored.
template <int DT, int KB>
__device__ __forceinline__ void issue_stage(GStage<DT, KB>& st, const GArgs& g, int chunk, int wave, int lane,
                                            int n0, int m0) {
    using P = GPlan<DT, KB>;
    constexpr int QB = GStage<DT, KB>::QB;
    const int b0 = g.kb0 + chunk * KB;
#pragma unroll
    for (int k = 0; k < P::PER_WAVE; ++k) {
        const int ins = NW * k + wave;  // uniform per wave
        if (ins >= P::I_TOTAL) break;
        const void* src;
        lds_ptr_t dst;
        if (ins < P::I_A) {
            const int p = ins * 64 + lane;
            constexpr int per_blk = TILE * QB / 16;
            const int blk = p / per_blk, rem = p - blk * per_blk;
            const int row = QB == 32 ? rem >> 1 : rem, half = QB == 32 ? rem & 1 : 0;
            const int n = n0 + row < g.rows ? n0 + row : g.rows - 1;
            const int b = b0 + blk < g.nb ? b0 + blk : g.nb - 1;
            src = g.qs + (size_t)n * g.qrow + (size_t)b * QB + 16 * half;
            dst = (lds_ptr_t)&st.A[ins * 64 * 16];
        } else if (ins < P::I_A + P::I_B) {
            const int i = ins - P::I_A;
            const int p = i * 64 + lane;
            const int blk = p / (TILE * 2), rem = p - blk * TILE * 2;
            const int tok = rem >> 1, half = rem & 1;
            const int m = m0 + tok < g.n_tok ? m0 + tok : g.n_tok - 1;
            const int b = b0 + blk < g.nb ? b0 + blk : g.nb - 1;
            src = g.aq + (size_t)m * g.cols + (size_t)b * 32 + 16 * half;
            dst = (lds_ptr_t)&st.B[i * 64 * 16];
        } else {
            // Scale tables, [blk][TILE] f32 each: TILE / 4 pieces of 4 floats per block.
            const int i = ins - P::I_A - P::I_B;
            const int table = i / P::I_S, j = i - table * P::I_S;
            const int p = j * 64 + lane;
            const int blk = p / (TILE / 4), r4 = (p - blk * (TILE / 4)) * 4;
            const int b = b0 + blk < g.nb ? b0 + blk : g.nb - 1;
            float* base;
            if (table == 0) {
                src = g.swT + (size_t)b * g.rows_pad + n0 + r4;
                base = st.SW;
            } else if (table == 1) {
                src = g.sxT + (size_t)b * g.tok_pad + m0 + r4;
                base = st.SX;
            } else if (table == 2) {
                src = g.swT + (size_t)g.nb * g.rows_pad + (size_t)b * g.rows_pad + n0 + r4;
                base = st.BI;
            } else {
                src = g.sxT + (size_t)g.nb * g.tok_pad + (size_t)b * g.tok_pad + m0 + r4;
                base = st.SXQ;
            }
            dst = (lds_ptr_t)&base[j * 64 * 4];
        }
        __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
    }
}

// Two outer products u_0 v_0^T and u_1 v_1^T of 32-vectors, exact in f32
// (the factors are BF16 values, so every product has at most 16 significant
// bits), each laid out like the i8 MFMA's result: one
// v_mfma_f32_32x32x1_2b_f32, lane l giving u_{l/32}[l%32] and v_{l/32}[l%32];
// result registers 16 b .. 16 b + 15 hold product b.
__device__ __forceinline__ v32f outer32x2(float u, float v) {
    const v32f z = {};
    return __builtin_amdgcn_mfma_f32_32x32x1f32(u, v, z, 0, 0, 0);
}

// One wave's 32 x 32 tile (rows rowA.., tokens colB..) over the stage's
// blocks, two at a time: lanes 0-31 read the scales of the first block of a
// pair, lanes 32-63 those of the second.
template <int DT, int KB>
__device__ __forceinline__ void compute_stage(const GStage<DT, KB>& st, v16f& acc, int nblk, int rowA, int colB, int h,
                                              int c) {
    constexpr int QB = GStage<DT, KB>::QB;
    static_assert(KB % 2 == 0, "blocks go in pairs");
#pragma unroll
    for (int jp = 0; jp < KB; jp += 2) {
        if (jp >= nblk) break;
        const int jh = jp + h;  // this lane's block for the scale products
        const v32f S = outer32x2(st.SW[jh * TILE + rowA + c], st.SX[jh * TILE + colB + c]);  // s_w[n] s_x[m]
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const int j = jp + jj;
            if (j >= nblk) break;
            const int4 bq = *(const int4*)&st.B[(j * TILE + colB + c) * 32 + 16 * h];
            int4 a;
            if (DT == 1) {
                a = *(const int4*)&st.A[(j * TILE + rowA + c) * QB + 16 * h];
            } else {
                const int4 q = *(const int4*)&st.A[(j * TILE + rowA + c) * QB];
                const int sh = 4 * h, mk = 0x0f0f0f0f;
                a.x = (int)((unsigned)q.x >> sh) & mk;
                a.y = (int)((unsigned)q.y >> sh) & mk;
                a.z = (int)((unsigned)q.z >> sh) & mk;
                a.w = (int)((unsigned)q.w >> sh) & mk;
            }
            const v16i z = {};
            const v16i P = __builtin_amdgcn_mfma_i32_32x32x32_i8(v4i{a.x, a.y, a.z, a.w}, v4i{bq.x, bq.y, bq.z, bq.w},
                                                                 z, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[r] = __builtin_fmaf((float)P[r], S[16 * jj + r], acc[r]);
        }
        if (DT == 2) {
            // Bias term of the pair: acc += sum_j bias[n, j] (s_x sum q_x)[m, j],
            // lane l giving bias[row l%32] and s_x sum q_x[token l%32] of block
            // jp + l/32 (zero past the stage's blocks).
            const float bi = jh < nblk ? st.BI[jh * TILE + rowA + c] : 0.0f;
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(bi, st.SXQ[jh * TILE + colB + c], acc, 0, 0, 0);
        }
    }
}

// One step of the ring: chunk c is in stage `cur`; chunk c + 2 goes into
// `nxt`, the stage chunk c - 1 was computed from.
template <int DT, int KB>
__device__ __forceinline__ void pipeline_step(GStage<DT, KB>& cur, GStage<DT, KB>& nxt, const GArgs& g, int c,
                                              int nchunks, v16f& acc, double (&tot)[16], int wave, int lane, int n0,
                                              int m0, int wn, int wm, int h) {
    using P = GPlan<DT, KB>;
    if (c >= nchunks) return;
    // This wave's loads of chunk c are done once at most chunk c + 1's are outstanding.
    if (c + 1 >= nchunks)
        __builtin_amdgcn_s_waitcnt(NNH_VMCNT(0));
    else if (P::full(wave))
        __builtin_amdgcn_s_waitcnt(NNH_VMCNT(P::PER_WAVE));
    else
        __builtin_amdgcn_s_waitcnt(NNH_VMCNT(P::PER_WAVE - 1));
    // Every wave's loads of chunk c have landed, and every wave is done with
    // chunk c - 1. A bare barrier: __syncthreads() would also wait for the
    // loads still in flight for chunks c + 1 and c + 2.
    __builtin_amdgcn_s_barrier();
    if (c + 2 < nchunks) issue_stage<DT, KB>(nxt, g, c + 2, wave, lane, n0, m0);
    const int left = g.kb1 - g.kb0 - c * KB;
    const int nblk = left < KB ? left : KB;
    compute_stage<DT, KB>(cur, acc, nblk, wn * 32, wm * 32, h, lane & 31);
    // The f32 sum goes into the f64 total every 8 blocks and at the end.
    if ((c & 1) || c + 1 == nchunks) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            tot[r] += (double)acc[r];
            acc[r] = 0.0f;
        }
    }
}

// A wave's 32 x 32 result tile turned around in LDS (`wout`, 4 KB), as
// [token][row ^ token] f32: the XOR spreads both passes over the banks.
// tile_put writes result register r of the lane; tile_store then writes
// 32-float runs of y rows.
__device__ __forceinline__ void tile_put(float* wout, int r, double v, int h, int c) {
    const int row = (r / 4) * 8 + 4 * h + (r % 4);
    wout[c * 32 + (row ^ c)] = (float)v;
}

__device__ __forceinline__ void tile_store(const float* wout, int n0, int m0, int h, int c, int rows, int n_tok,
                                           float* __restrict__ y, size_t y_stride) {
    const int n = n0 + c;
#pragma unroll 4
    for (int k = 0; k < 16; ++k) {
        const int t = 2 * k + h;
        const int m = m0 + t;
        const float v = wout[t * 32 + (c ^ t)];
        if (n < rows && m < n_tok) y[(size_t)m * y_stride + n] = v;
    }
}

__device__ __forceinline__ void store_tile(float* wout, const double (&acc)[16], int n0, int m0, int h, int c,
                                           int rows, int n_tok, float* __restrict__ y, size_t y_stride) {
#pragma unroll
    for (int r = 0; r < 16; ++r) tile_put(wout, r, acc[r], h, c);
    tile_store(wout, n0, m0, h, c, rows, n_tok, y, y_stride);
}

template <int DT, int KB>
__global__ __launch_bounds__(NW * 64) void gemm_i8_kernel(GArgs g, float* __restrict__ y, size_t y_stride) {
    // Three distinct objects, not one array: the compiler then sees that the
    // loads into one stage do not alias the reads of another, and inserts no
    // wait for the loads in flight before reading the current stage.
    __shared__ __attribute__((aligned(16))) GStage<DT, KB> s0, s1, s2;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int h = lane >> 5, c = lane & 31;
    const int wn = wave / WM, wm = wave % WM;
    // Workgroups go round-robin to the 8 XCDs (one L2 each); renumber them so
    // that each XCD takes a contiguous range of (row tile, split) pairs and
    // reads those weights once, for every token tile.
    const int total = gridDim.x, per = total / 8, rem = total % 8;
    const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
    const int id = xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
    const int mt = id % g.mtiles, rest = id / g.mtiles;
    const int split = rest % g.splits, rt = rest / g.splits;
    const int n0 = rt * TILE, m0 = mt * TILE;
    GArgs gl = g;
    gl.kb0 = (int)((long)split * g.nb / g.splits);
    gl.kb1 = (int)((long)(split + 1) * g.nb / g.splits);
    const int nchunks = (gl.kb1 - gl.kb0 + KB - 1) / KB;

    double tot[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) tot[r] = 0.0;
    v16f acc = {};

    issue_stage<DT, KB>(s0, gl, 0, wave, lane, n0, m0);
    if (nchunks > 1) issue_stage<DT, KB>(s1, gl, 1, wave, lane, n0, m0);
    for (int ch = 0; ch < nchunks; ch += 3) {
        pipeline_step<DT, KB>(s0, s2, gl, ch, nchunks, acc, tot, wave, lane, n0, m0, wn, wm, h);
        pipeline_step<DT, KB>(s1, s0, gl, ch + 1, nchunks, acc, tot, wave, lane, n0, m0, wn, wm, h);
        pipeline_step<DT, KB>(s2, s1, gl, ch + 2, nchunks, acc, tot, wave, lane, n0, m0, wn, wm, h);
    }

    if (g.splits > 1) {
        // Partial tile to the workspace, register-major: 512-byte runs per store.
        double* p = g.ws + (((size_t)split * g.tiles + rt * g.mtiles + mt) * NW + wave) * 1024 + lane;
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r * 64] = tot[r];
        return;
    }
    static_assert(NW == 16 && sizeof(GStage<DT, KB>) >= 8 * 32 * 32 * sizeof(float),
                  "output staging: eight 4 KB wave tiles per stage, two stages");
    __syncthreads();  // every wave is done with the ring (no loads remain in flight)
    float* wout = (wave < 8 ? (float*)&s0 : (float*)&s1) + (wave % 8) * 32 * 32;
    store_tile(wout, tot, n0 + wn * 32, m0 + wm * 32, h, c, g.rows, g.n_tok, y, y_stride);
}

// y = the sum of the split-K partial tiles, in split order (f64), rounded
// once. One 64-lane workgroup per wave tile of the GEMM; four result
// registers at a time, their partials loaded for every split before the
// first add so the latencies overlap.
__global__ __launch_bounds__(64) void gemm_reduce_kernel(const double* __restrict__ ws, int splits, int tiles,
                                                         int mtiles, int rows, int n_tok, float* __restrict__ y,
                                                         size_t y_stride) {
    __shared__ float out[32 * 32];
    const int lane = threadIdx.x, h = lane >> 5, c = lane & 31;
    const int tile = blockIdx.x / NW, wave = blockIdx.x % NW;
    const double* base = ws + ((size_t)tile * NW + wave) * 1024 + lane;
    const size_t split_stride = (size_t)tiles * NW * 1024;
#pragma unroll 1
    for (int r0 = 0; r0 < 16; r0 += 4) {
        double p[GEMM_MAX_SPLITS][4];
#pragma unroll
        for (int sp = 0; sp < GEMM_MAX_SPLITS; ++sp)
#pragma unroll
            for (int r = 0; r < 4; ++r) p[sp][r] = sp < splits ? base[sp * split_stride + (r0 + r) * 64] : 0.0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            double s = 0.0;
#pragma unroll
            for (int sp = 0; sp < GEMM_MAX_SPLITS; ++sp)
                if (sp < splits) s += p[sp][r];
            tile_put(out, r0 + r, s, h, c);
        }
    }
    const int n0 = (tile / mtiles) * TILE + (wave / WM) * 32, m0 = (tile % mtiles) * TILE + (wave % WM) * 32;
    tile_store(out, n0, m0, h, c, rows, n_tok, y, y_stride);
}

// swT[b][n] = f32(scale[n][b]) and, for Q4, the biases in a second table
// after it; rows padded to a multiple of TILE with zeros.
__global__ void gemm_scales_kernel(const uint16_t* __restrict__ sc, const uint16_t* __restrict__ bi,
                                   float* __restrict__ swT, int rows, int rows_pad, int nb) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t per = (size_t)rows_pad * nb;
    const int tables = bi ? 2 : 1;
    if (idx >= per * tables) return;
    const int tbl = (int)(idx / per);
    const size_t r = idx - tbl * per;
    const int b = (int)(r / rows_pad), n = (int)(r - (size_t)b * rows_pad);
    const uint16_t* src = tbl == 0 ? sc : bi;
    swT[idx] = n < rows ? bf16f(src[(size_t)n * nb + b]) : 0.0f;
}

}  // namespace

int gemm_rows_pad(int rows) { return (rows + TILE - 1) / TILE * TILE; }
int gemm_tok_pad(int n_tok) { return (n_tok + TILE - 1) / TILE * TILE; }

void launch_gemm_scales(const uint16_t* sc, const uint16_t* bi, float* swT, int rows, int nb, hipStream_t st) {
    const int rp = gemm_rows_pad(rows);
    const size_t n = (size_t)rp * nb * (bi ? 2 : 1);
    gemm_scales_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(sc, bi, swT, rows, rp, nb);
}

// Blocks per ring stage.
constexpr int GEMM_KB = 4;


// Split-K factor: small tile grids are split along K until they cover the
// 256 CUs (one workgroup each), keeping at least two ring chunks per split.
int gemm_splits(int rows, int nb, int n_tok) {
    const int tiles = ceil_div(rows, TILE) * ceil_div(n_tok, TILE);
    if (tiles >= 192) return 1;
    int sp = (256 + tiles / 2) / tiles;
    const int most = nb / (2 * GEMM_KB);
    if (sp > most) sp = most;
    if (sp > GEMM_MAX_SPLITS) sp = GEMM_MAX_SPLITS;
    return sp < 1 ? 1 : sp;
}

size_t gemm_workspace_bytes(int rows, int nb, int n_tok) {
    const int sp = gemm_splits(rows, nb, n_tok);
    if (sp == 1) return 0;
    return (size_t)sp * ceil_div(rows, TILE) * ceil_div(n_tok, TILE) * TILE * TILE * sizeof(double);
}

void launch_gemm_i8(int dtype, const uint8_t* qs, const float* swT, const int8_t* aq, const float* sxT, int rows,
                    int nb, int n_tok, float* y, size_t y_stride, double* ws, hipStream_t st) {
    GArgs g;
    g.qs = qs;
    g.swT = swT;
    g.aq = aq;
    g.sxT = sxT;
    g.ws = ws;
    g.rows = rows;
    g.rows_pad = gemm_rows_pad(rows);
    g.nb = nb;
    g.n_tok = n_tok;
    g.tok_pad = gemm_tok_pad(n_tok);
    g.mtiles = ceil_div(n_tok, TILE);
    g.tiles = g.mtiles * ceil_div(rows, TILE);
    g.splits = gemm_splits(rows, nb, n_tok);
    g.kb0 = 0;
    g.kb1 = nb;
    g.cols = (size_t)nb * 32;
    g.qrow = dtype == 1 ? g.cols : g.cols / 2;
    const dim3 grid(g.tiles * g.splits), block(NW * 64);
    if (dtype == 1)
        gemm_i8_kernel<1, GEMM_KB><<<grid, block, 0, st>>>(g, y, y_stride);
    else
        gemm_i8_kernel<2, GEMM_KB><<<grid, block, 0, st>>>(g, y, y_stride);
    if (g.splits > 1)
        gemm_reduce_kernel<<<g.tiles * NW, 64, 0, st>>>(ws, g.splits, g.tiles, g.mtiles, rows, n_tok, y, y_stride);
}

}  // namespace nnh
