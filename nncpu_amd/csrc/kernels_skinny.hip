// The int8 matmul for a few activation vectors (4..16: batched speculative
// verify, short prompts) on the matrix unit: a weight stream with a
// 32-token MFMA.
//
// One v_mfma_i32_32x32x32_i8 per (32 weight rows, block): A = the
// activations (MFMA rows i = tokens, padded to 32), B = the weights (MFMA
// columns j = weight rows). Result element (i, j) sits in lane j + 32h,
// register r with i = (r/4)*8 + 4h + r%4, so tokens 0..7 are registers 0..3
// and tokens 8..15 registers 4..7 of every lane: only NR = 4 or 8 registers
// per lane carry real outputs, and the scaling epilogue runs on those alone.
// The block dot products are exact; the epilogue is the GEMM's (exact scale
// products from a two-block f32 outer-product MFMA, f64 accumulation), so
// every output is within one f32 ulp of the exact sum.
//
// Workgroup: 16 waves on 32 weight rows. Weights, activations (tokens
// 0..15) and scales stream through a ring of three LDS stages of 16 blocks,
// filled by direct global -> LDS loads in which consecutive lanes read
// consecutive 16-byte pieces of a row (coalesced), placed XOR-swizzled so
// the MFMA operand reads are free of bank conflicts. All 16 waves issue the
// loads, two per stage each (a wave keeps only a few loads in flight: the
// same bytes over 16 waves arrive about twice as fast as over 4, measured);
// the first 8 waves compute two blocks of a stage each, and their partial
// sums meet in LDS, added in wave order.
// Matrices with few row groups are split along K over several workgroups
// as well; those partials go to a workspace (f64) and a second kernel adds
// them in split order.

#include "common.h"

namespace nnh {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

constexpr int SK_W = 16;          // waves per workgroup (8 where registers are short): all issue loads
constexpr int SK_CW = 8;          // of which the first SK_CW compute (2 blocks of a stage each)
constexpr int SK_KC = 16;         // blocks per ring stage: 4 per wave
constexpr int SK_MAX_SPLITS = 8;  // K-split workgroups per row group

struct KArgs {
    const uint8_t* qs;  // weights, nncpu row-major quants
    const float* swT;   // [nb][rows_pad] weight scales; Q4 biases follow at + nb * rows_pad
    const int8_t* aq;   // activation quants [n_tok][cols]
    const float* sxT;   // [nb][tok_pad] activation scales, then [nb][tok_pad] scale * sum(q)
    double* ws;         // K-split partials [split][16][rows_pad] (ksplit > 1)
    int rows, rows_pad, nb, n_tok, tok_pad, ksplit;
    size_t qrow, cols;
};

// One ring stage: SK_KC blocks of the workgroup's 32 weight rows and of
// tokens 0..15, with their scales. Quant rows are XOR-swizzled at 16-byte
// granularity (piece q of row r at position q ^ (r % 16)), so the MFMA
// operand reads (32 rows, one piece each) hit 16 distinct bank groups.
template <int DT, int NW, int TOK>
struct KStage {
    static constexpr int QB = DT == 1 ? 32 : 16;  // weight bytes per row and block
    static constexpr int WROW = SK_KC * QB;       // bytes per staged weight row
    static constexpr int XROW = SK_KC * 32;       // bytes per staged token row
    // Load instructions that fill a stage, and the padding that rounds them
    // up to a whole number per wave (those land in PAD and are never read).
    static constexpr int I_REAL = (32 * WROW + TOK * XROW + SK_KC * 32 * 4 * (DT == 2 ? 4 : 2)) / 1024;
    static constexpr int I_PAD = (NW - I_REAL % NW) % NW;
    uint8_t W[32 * WROW];
    int8_t X[TOK * XROW];  // tokens 0..TOK-1
    float SW[SK_KC * 32];  // [blk][row]
    float SX[SK_KC * 32];  // [blk][token]
    float BI[DT == 2 ? SK_KC * 32 : 4];
    float SXQ[DT == 2 ? SK_KC * 32 : 4];
    uint8_t PAD[I_PAD > 0 ? I_PAD * 1024 : 16];
};

template <int DT, int NW, int TOK>
struct KPlan {
    static constexpr int I_W = 32 * KStage<DT, NW, TOK>::WROW / 1024;      // 1 KB per load instruction
    static constexpr int I_X = TOK * KStage<DT, NW, TOK>::XROW / 1024;
    static constexpr int I_S = SK_KC * 32 * 4 / 1024;              // per scale table
    static constexpr int N_S = (DT == 2 ? 4 : 2) * I_S;
    static constexpr int I_TOTAL = I_W + I_X + N_S + KStage<DT, NW, TOK>::I_PAD;
    static constexpr int PER_WAVE = I_TOTAL / NW;
    static_assert(I_TOTAL % NW == 0 && I_W + I_X + N_S == KStage<DT, NW, TOK>::I_REAL, "loads split evenly over the waves");
    static_assert(KStage<DT, NW, TOK>::WROW / 16 >= 16 && KStage<DT, NW, TOK>::XROW / 16 >= 16, "swizzle needs 16 pieces per row");
    static_assert(3 * PER_WAVE < 64, "vmcnt holds at most 63");
};

// The load feeding staged position `pos` (16-byte units) of a swizzled
// region with `ppr` pieces per row: row pos / ppr, global piece (pos % ppr)
// ^ (row % 16). Consecutive lanes cover whole rows: coalesced.
__device__ __forceinline__ void swz_src(int pos, int ppr, int& row, int& piece) {
    row = pos / ppr;
    piece = (pos - row * ppr) ^ (row & 15);
}

template <int DT, int NW, int TOK>
__device__ __forceinline__ void k_issue(KStage<DT, NW, TOK>& st, const KArgs& g, int b0, int kb1, int wave, int lane, int n0) {
    using P = KPlan<DT, NW, TOK>;
    constexpr int QB = KStage<DT, NW, TOK>::QB;
#pragma unroll
    for (int k = 0; k < P::PER_WAVE; ++k) {
        const int ins = NW * k + wave;  // uniform per wave
        const void* src;
        lds_ptr_t dst;
        if (ins < P::I_W) {
            int row, piece;
            swz_src(ins * 64 + lane, KStage<DT, NW, TOK>::WROW / 16, row, piece);
            const int n = n0 + row < g.rows ? n0 + row : g.rows - 1;
            // Pieces past the range repeat the last block (never used).
            int b = b0 + piece * 16 / QB;
            const int within = piece * 16 - (piece * 16 / QB) * QB;
            if (b >= kb1) b = kb1 - 1;
            src = g.qs + (size_t)n * g.qrow + (size_t)b * QB + within;
            dst = (lds_ptr_t)&st.W[ins * 1024];
        } else if (ins < P::I_W + P::I_X) {
            const int i = ins - P::I_W;
            int row, piece;
            swz_src(i * 64 + lane, KStage<DT, NW, TOK>::XROW / 16, row, piece);
            const int t = row < g.n_tok ? row : g.n_tok - 1;
            int b = b0 + (piece >> 1);
            if (b >= kb1) b = kb1 - 1;
            src = g.aq + (size_t)t * g.cols + (size_t)b * 32 + 16 * (piece & 1);
            dst = (lds_ptr_t)&st.X[i * 1024];
        } else if (ins >= KStage<DT, NW, TOK>::I_REAL) {
            // Padding: one valid 16-byte source for every lane, into PAD.
            src = g.aq;
            dst = (lds_ptr_t)&st.PAD[(ins - KStage<DT, NW, TOK>::I_REAL) * 1024];
        } else {
            // Scale tables, [blk][32] f32: 8 pieces of 4 floats per block.
            const int i = ins - P::I_W - P::I_X;
            const int table = i / P::I_S, j = i - table * P::I_S;
            const int p = j * 64 + lane;
            const int blk = p >> 3, r4 = (p & 7) * 4;
            int b = b0 + blk;
            if (b >= kb1) b = kb1 - 1;
            float* base;
            if (table == 0) {
                src = g.swT + (size_t)b * g.rows_pad + n0 + r4;
                base = st.SW;
            } else if (table == 1) {
                src = g.sxT + (size_t)b * g.tok_pad + r4;
                base = st.SX;
            } else if (table == 2) {
                src = g.swT + (size_t)g.nb * g.rows_pad + (size_t)b * g.rows_pad + n0 + r4;
                base = st.BI;
            } else {
                src = g.sxT + (size_t)g.nb * g.tok_pad + (size_t)b * g.tok_pad + r4;
                base = st.SXQ;
            }
            dst = (lds_ptr_t)&base[j * 256];
        }
        __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
    }
}

// This wave's blocks 4w..4w+3 of the stage (those below nblk), in pairs for
// the two-block scale outer products.
template <int DT, int NR, int NW>
__device__ __forceinline__ void k_compute(const KStage<DT, NW, 2 * NR>& st, double (&acc)[NR], int nblk, int wave, int h,
                                          int c) {
    constexpr int QB = KStage<DT, NW, 2 * NR>::QB;
    const int tc = c < 2 * NR ? c : 2 * NR - 1;  // unstaged tokens: any staged row (results unused)
    {
        const int j0 = 2 * wave;  // this wave's pair of the stage's blocks
        if (j0 >= nblk) return;
        const int jh = j0 + h;  // this lane's block of the pair for the scale products
        const v32f z = {};
        // s_x[token i] * s_w[row j] for blocks j0 and j0 + 1, exact in f32.
        const v32f S = __builtin_amdgcn_mfma_f32_32x32x1f32(st.SX[jh * 32 + c], st.SW[jh * 32 + c], z, 0, 0, 0);
        v32f Q;
        if (DT == 2) Q = __builtin_amdgcn_mfma_f32_32x32x1f32(st.SXQ[jh * 32 + c], 1.0f, z, 0, 0, 0);
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const int j = j0 + jj;
            if (j >= nblk) break;
            // Weights: row c, piece (QB == 32 ? 2j + h : j); activations: token tc, piece 2j + h.
            const int wq = QB == 32 ? 2 * j + h : j;
            int4 w = *(const int4*)&st.W[c * KStage<DT, NW, 2 * NR>::WROW + 16 * (wq ^ (c & 15))];
            if (DT == 2) {
                const int sh = 4 * h, mk = 0x0f0f0f0f;
                w.x = (int)((unsigned)w.x >> sh) & mk;
                w.y = (int)((unsigned)w.y >> sh) & mk;
                w.z = (int)((unsigned)w.z >> sh) & mk;
                w.w = (int)((unsigned)w.w >> sh) & mk;
            }
            const int4 a = *(const int4*)&st.X[tc * KStage<DT, NW, 2 * NR>::XROW + 16 * ((2 * j + h) ^ (tc & 15))];
            const v16i zi = {};
            const v16i P = __builtin_amdgcn_mfma_i32_32x32x32_i8(v4i{a.x, a.y, a.z, a.w}, v4i{w.x, w.y, w.z, w.w},
                                                                 zi, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < NR; ++r) acc[r] = __builtin_fma((double)P[r], (double)S[16 * jj + r], acc[r]);
            if (DT == 2) {
                const double bi = (double)st.BI[j * 32 + c];  // bias[row] * (s_x sum q_x)[token], exact in f64
#pragma unroll
                for (int r = 0; r < NR; ++r) acc[r] = __builtin_fma(bi, (double)Q[16 * jj + r], acc[r]);
            }
        }
    }
}

// Chunks 0..2 are issued at the start (every stage of the ring); after
// that, chunk c + 2 is issued at step c into the stage chunk c - 1 used.
template <int DT, int NR, int NW>
__device__ __forceinline__ void k_step(KStage<DT, NW, 2 * NR>& cur, KStage<DT, NW, 2 * NR>& nxt, const KArgs& g, int c, int nchunks, int kb0,
                                       int kb1, double (&acc)[NR], int wave, int lane, int n0) {
    if (c >= nchunks) return;
    // This wave's loads of chunk c are done once only later chunks' are
    // outstanding: chunks 1 and 2 at step 0, chunk c + 1 after that.
    if (c == 0 && nchunks > 2)
        __builtin_amdgcn_s_waitcnt(NNH_VMCNT((2 * KPlan<DT, NW, 2 * NR>::PER_WAVE)));
    else if (c + 1 < nchunks)
        __builtin_amdgcn_s_waitcnt(NNH_VMCNT((KPlan<DT, NW, 2 * NR>::PER_WAVE)));
    else
        __builtin_amdgcn_s_waitcnt(NNH_VMCNT(0));
    __builtin_amdgcn_s_barrier();  // every wave's loads landed; every wave done with chunk c - 1
    if (c >= 1 && c + 2 < nchunks) k_issue<DT, NW, 2 * NR>(nxt, g, kb0 + (c + 2) * SK_KC, kb1, wave, lane, n0);
    const int left = kb1 - kb0 - c * SK_KC;
    if (wave < SK_CW) k_compute<DT, NR, NW>(cur, acc, left < SK_KC ? left : SK_KC, wave, lane >> 5, lane & 31);
}

template <int DT, int NR, int NW>
__global__ __launch_bounds__(NW * 64) void skinny_i8_kernel(KArgs g, float* __restrict__ y, size_t y_stride) {
    // Distinct objects, so the compiler sees that loads into one stage do not
    // alias reads of another (one array would make it wait for every load).
    __shared__ __attribute__((aligned(16))) KStage<DT, NW, 2 * NR> s0, s1, s2;
    __shared__ double red[SK_CW][NR][64];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int rg = blockIdx.x / g.ksplit, ks = blockIdx.x % g.ksplit;
    const int n0 = rg * 32;
    const int kb0 = (int)((long)ks * g.nb / g.ksplit), kb1 = (int)((long)(ks + 1) * g.nb / g.ksplit);
    const int nchunks = (kb1 - kb0 + SK_KC - 1) / SK_KC;

    double acc[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = 0.0;
    if (nchunks > 0) k_issue<DT, NW, 2 * NR>(s0, g, kb0, kb1, wave, lane, n0);
    if (nchunks > 1) k_issue<DT, NW, 2 * NR>(s1, g, kb0 + SK_KC, kb1, wave, lane, n0);
    if (nchunks > 2) k_issue<DT, NW, 2 * NR>(s2, g, kb0 + 2 * SK_KC, kb1, wave, lane, n0);
    for (int c = 0; c < nchunks; c += 3) {
        k_step<DT, NR, NW>(s0, s2, g, c, nchunks, kb0, kb1, acc, wave, lane, n0);
        k_step<DT, NR, NW>(s1, s0, g, c + 1, nchunks, kb0, kb1, acc, wave, lane, n0);
        k_step<DT, NR, NW>(s2, s1, g, c + 2, nchunks, kb0, kb1, acc, wave, lane, n0);
    }

    if (wave < SK_CW) {
#pragma unroll
        for (int r = 0; r < NR; ++r) red[wave][r][lane] = acc[r];
    }
    __syncthreads();
    // Thread (r, l) of the first NR waves finishes result register r of lane l.
    static_assert(NR <= NW, "one round");
    const int l = tid & 63;
    const int row = n0 + (l & 31);
    {
        const int r = tid >> 6;
        if (r >= NR) return;
        double s = 0.0;
#pragma unroll
        for (int w = 0; w < SK_CW; ++w) s += red[w][r][l];
        const int i = (r / 4) * 8 + 4 * (l >> 5) + (r % 4);  // token
        if (i < g.n_tok && row < g.rows) {
            if (g.ksplit == 1)
                y[(size_t)i * y_stride + row] = (float)s;
            else
                g.ws[((size_t)ks * 16 + i) * g.rows_pad + row] = s;
        }
    }
}

// y = the sum of the K-split partials in split order (f64), rounded once.
// All partials are loaded before the first add, so their latencies overlap.
__global__ void skinny_reduce_kernel(const double* __restrict__ ws, int ksplit, int rows, int rows_pad, int n_tok,
                                     float* __restrict__ y, size_t y_stride) {
    const int row = blockIdx.x * blockDim.x + threadIdx.x, i = blockIdx.y;
    if (row >= rows) return;
    double p[SK_MAX_SPLITS];
#pragma unroll
    for (int k = 0; k < SK_MAX_SPLITS; ++k) p[k] = k < ksplit ? ws[((size_t)k * 16 + i) * rows_pad + row] : 0.0;
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < SK_MAX_SPLITS; ++k)
        if (k < ksplit) s += p[k];
    y[(size_t)i * y_stride + row] = (float)s;
}

}  // namespace

// K-split over workgroups when the row groups alone do not cover the CUs;
// each split keeps at least one full ring stage.
int skinny_splits(int rows, int nb) {
    const int groups = ceil_div(rows, 32);
    if (groups >= 160) return 1;
    int ks = 256 / groups;  // one workgroup per CU (the ring takes most of the LDS)
    const int most = nb / SK_KC;
    if (ks > most) ks = most;
    if (ks > SK_MAX_SPLITS) ks = SK_MAX_SPLITS;
    return ks < 1 ? 1 : ks;
}

size_t skinny_workspace_bytes(int rows, int nb) {
    const int ks = skinny_splits(rows, nb);
    return ks == 1 ? 0 : (size_t)ks * 16 * gemm_rows_pad(rows) * sizeof(double);
}

void launch_skinny_i8(int dtype, const uint8_t* qs, const float* swT, const int8_t* aq, const float* sxT, int rows,
                      int nb, int n_tok, float* y, size_t y_stride, double* ws, hipStream_t st) {
    KArgs g;
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
    g.ksplit = skinny_splits(rows, nb);
    g.cols = (size_t)nb * 32;
    g.qrow = dtype == 1 ? g.cols : g.cols / 2;
    const dim3 grid(ceil_div(rows, 32) * g.ksplit);
    // Q4 with 16 tokens needs more registers than 16 waves leave a lane: 8 waves there.
#define NNH_SK(DT, NR, NW) skinny_i8_kernel<DT, NR, NW><<<grid, NW * 64, 0, st>>>(g, y, y_stride)
    if (dtype == 1) {
        if (n_tok <= 8) NNH_SK(1, 4, SK_W); else NNH_SK(1, 8, SK_W);
    } else {
        if (n_tok <= 8) NNH_SK(2, 4, SK_W); else NNH_SK(2, 8, SK_W / 2);
    }
#undef NNH_SK
    if (g.ksplit > 1)
        skinny_reduce_kernel<<<dim3(ceil_div(rows, 256), n_tok), 256, 0, st>>>(ws, g.ksplit, rows, g.rows_pad, n_tok, y,
                                                                               y_stride);
}

}  // namespace nnh
