// The MX int8 path: activations quantized to int8 blocks of 32 with a
// power-of-two scale (the OCP MXINT8 block: 32 int8 values and one shared
// exponent), and the GEMM for many vectors (prefill, batched verify) that
// this makes cheap on the matrix unit:
//
//   y[m][n] = sum_b s_w[n,b] * P'_b[m][n]     (+ Q4: sum_b bias[n,b] X[m,b])
//   P'_b[m][n] = sum_k (q_x[m,32b+k] 2^E[m,b]) * q_w[n,32b+k]
//   X[m,b] = 2^E[m,b] * sum_k q_x[m,32b+k]
//
// With a power-of-two activation scale, q_x 2^E is a BF16 value exactly
// (7 significant bits), and so is every weight quant (Q8 -127..127, Q4
// 0..15). A BF16 MFMA therefore forms P'_b exactly: every product is an
// integer times 2^E, and every partial sum of a block stays below 2^19 2^E,
// inside f32's 24 bits, whatever order the hardware adds in. So
// P'_b = 2^E P_b with P_b the exact int32 block dot product, already in f32,
// and the epilogue is ONE fma per output and block by the weight scale, which
// is a single value per lane because the lane layout puts one weight row in
// each lane. (nncpu's BF16 activation scales would need the scale product
// s_w s_x per output and block: a conversion, a product and an fma.)
//
// The Q4 bias term is an outer-product sum over blocks, so it runs on the
// matrix unit too: X split into two BF16 limbs (hi = X's top 8 significant
// bits, lo = the rest, both exact), and one BF16 MFMA of K = 16 per 8 blocks
// (4 blocks x 2 limbs per lane half) against the biases, each stored twice.
//
// Accumulation: the f32 sum of a chunk of FOLD_GROUPS x 8 blocks is added
// into an f32 total (registers hold four 32 x 32 tiles per wave, no room
// for f64 totals), so each output is within the chunk's f32 roundings plus
// one rounding per fold of its exact value; split tiles' partial totals are
// added in f64 and rounded once.
//
// Work split: the output is cut into 128-row x 256-token tiles and K into
// groups of 8 blocks. A "team" of workgroups, one per token tile, walks the
// same (row tile, group) units in the same order, so the team shares every
// weight stage through the L2 of its XCD. Whole row tiles go round-robin to
// the teams first (data-parallel rounds: every team at the same K group at
// about the same time, so the activations are shared in L2 too); the
// remaining row tiles' units are split evenly over the teams (stream-K), and
// a tile whose groups span two teams' shares gets partial tiles in a
// workspace, added in team order in f64 by gemm_mx_fixup_kernel
// (deterministic).
//
// Workgroup: 8 waves (2 per SIMD), wave (wm, wn) owns tokens 64 wm .. +63
// and rows 64 wn .. +63: 2 x 2 tiles of 32 x 32, each operand read from LDS
// serving two MFMAs. Operands stream through a ring of three LDS stages of
// 2 blocks (two in flight while one is computed), filled by direct
// global -> LDS loads (no staging registers) whose addresses are a scalar
// base plus a per-lane offset; 16-byte chunks of each 64-byte row are
// XOR-swizzled against bank conflicts. The weights arrive as nncpu's own
// quant bytes (Q8 1 byte, Q4 half a byte per weight, read in place from the
// uploaded split layout): each wave's direct load lands in a staging slice
// of the stage, and at the stage's turn the wave converts its slice to BF16
// (exact: the quants are small integers) into the stage's operand rows. A
// weight tile is reused by 256 tokens, so the conversion is a small VALU
// cost per MFMA, while the bytes streamed per weight are a half (Q8) or a
// quarter (Q4) of a BF16 copy's, and no such copy is kept.

#include "common.h"

namespace nnh {
namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int MX_NW = 8;           // waves per workgroup
constexpr int MX_KS = 2;           // blocks per ring stage
constexpr int MX_NS = 4;           // stages per 8-block group
constexpr int MX_GRP = 8;          // blocks per group
constexpr int MX_FOLD_GROUPS = 2;  // groups per f32 chunk before the f64 fold
constexpr int MX_TM_Q = 256;       // tokens per GEMM tile (the quantizer's xb tiles, = MX_TM)
constexpr int MX_MIN_UNITS = 2;    // groups per workgroup at least
static_assert(MX_KS * MX_NS == MX_GRP, "whole stages per group");

__device__ __forceinline__ int rint_sat_mx(float v) {
    float r = __builtin_rintf(v);
    if (!(r == r)) return 0;
    if (r >= 2147483648.0f) return 2147483647;
    if (r <= -2147483648.0f) return (int)0x80000000;
    return (int)r;
}

// ---- quantizer ---------------------------------------------------------------

// The exponent E of a block's power-of-two scale: the least E with
// 127 * 2^E >= amax, clamped to [-126, 127] (so 2^E is a normal f32 and
// BF16). amax = (1 + f) 2^e, 1 <= 1 + f < 2: 127 * 2^(e-6) = 1.984375 * 2^e
// covers it unless f > 0.984375 (mantissa bits above 0x7E0000), which needs
// e - 5. Exact on the bits, no rounding involved.
__device__ __forceinline__ int mx_exponent(float amax) {
    const uint32_t u = __float_as_uint(amax);
    const int be = (int)(u >> 23);
    if (be == 0) return -126;  // zero or subnormal amax
    int e = be - 127 - 6 + ((u & 0x7FFFFFu) > 0x7E0000u ? 1 : 0);
    return e < -126 ? -126 : (e > 127 ? 127 : e);
}

// One 32-lane half-wave per block of 32 values; blocks past nb (up to the
// group-padded nbp8) and tokens past n_tok (up to xl_tok, whole GEMM token
// tiles) only write zeros: the limbs of xl, and for tokens past n_tok the
// xb values.
__global__ __launch_bounds__(256) void quantize_mx_kernel(const float* __restrict__ x, size_t x_stride, int cols,
                                                          int n_tok, int nbp8, int8_t* __restrict__ q,
                                                          uint16_t* __restrict__ s, double* __restrict__ sx,
                                                          float* __restrict__ sxT, int tok_pad, int xl_tok,
                                                          uint16_t* __restrict__ xb, uint16_t* __restrict__ xl) {
    const int nb = cols >> 5;
    const int k = threadIdx.x & 31;
    const int blk = blockIdx.x * 8 + (threadIdx.x >> 5);
    if (blk >= nbp8 * xl_tok) return;  // uniform per half-wave
    const int t = blk / nbp8, b = blk - t * nbp8;
    // xb tiled: [token tile][block][token in tile][32], 16-byte chunks of a
    // row swizzled as the GEMM's LDS rows are (chunk c at c ^ ((row >> 2) & 3)).
    const int tt = t / MX_TM_Q, tr = t % MX_TM_Q;
    const size_t xe = (((size_t)tt * nb + b) * MX_TM_Q + tr) * 32 + (((k >> 3) ^ ((tr >> 2) & 3)) << 3) + (k & 7);
    if (b >= nb || t >= n_tok) {
        if (k < 2) xl[((size_t)t * nbp8 + b) * 2 + k] = 0;
        if (b < nb) xb[xe] = 0;
        return;
    }
    const float v = x[(size_t)t * x_stride + 32 * (size_t)b + k];
    // amax over the block, NaN skipped (as nncpu's encoder's `v.abs() > amax`).
    float a = fabsf(v);
    a = (a == a) ? a : 0.0f;
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) a = fmaxf(a, __shfl_xor(a, m, 32));
    const bool zero = !(a > 0.0f);
    const int E = mx_exponent(a);
    int qi = zero ? 0 : rint_sat_mx(__builtin_ldexpf(v, -E));  // v 2^-E: exact unless below 2^-126 (then |q| < 1)
    qi = qi < -127 ? -127 : (qi > 127 ? 127 : qi);
    int qsum = qi;
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) qsum += __shfl_xor(qsum, m, 32);
    const float scale = zero ? 0.0f : __uint_as_float((uint32_t)(E + 127) << 23);
    const size_t e = (size_t)t * cols + 32 * (size_t)b + k;
    q[e] = (int8_t)qi;
    // q 2^E as BF16: at most 7 significant bits, so the f32's low half is zero.
    xb[xe] = (uint16_t)(__float_as_uint((float)qi * scale) >> 16);
    if (k == 0) {
        const float X = scale * (float)qsum;  // exact: <= 12 significant bits
        s[(size_t)t * nb + b] = (uint16_t)(__float_as_uint(scale) >> 16);
        sx[2 * ((size_t)t * nb + b)] = (double)scale;
        sx[2 * ((size_t)t * nb + b) + 1] = (double)X;
        sxT[(size_t)b * tok_pad + t] = scale;
        sxT[(size_t)nb * tok_pad + (size_t)b * tok_pad + t] = X;
        // X = hi + lo, hi its top 8 significant bits, lo the rest (<= 4 bits).
        const uint32_t hb = __float_as_uint(X) & 0xFFFF0000u;
        const float lo = X - __uint_as_float(hb);
        xl[((size_t)t * nbp8 + b) * 2] = (uint16_t)(hb >> 16);
        xl[((size_t)t * nbp8 + b) * 2 + 1] = (uint16_t)(__float_as_uint(lo) >> 16);
    }
}

// ---- upload-time weight tables -------------------------------------------------

// Q4 biases twice per block, [rows_pad][nbp8][2], zero past nb and in the pad
// rows: the B operand of the bias MFMA, whose A operand holds X's limbs.
__global__ void mx_bias_kernel(const uint16_t* __restrict__ bi, uint16_t* __restrict__ wbi, int rows, int rows_pad,
                               int nb, int nbp8) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)rows_pad * nbp8) return;
    const int r = (int)(i / nbp8), b = (int)(i - (size_t)r * nbp8);
    const uint16_t v = b < nb && r < rows ? bi[(size_t)r * nb + b] : (uint16_t)0;
    wbi[2 * i] = v;
    wbi[2 * i + 1] = v;
}

// ---- GEMM ------------------------------------------------------------------------

constexpr int MX_TM = 256;  // tokens per tile
constexpr int MX_TN = 128;  // weight rows per tile
// 8 waves: 4 along tokens x 2 along rows, each 64 tokens x 64 rows (2 x 2
// MFMA tiles of 32 x 32).

struct MxStage {
    uint16_t A[MX_KS][MX_TM][32];  // activations, [blk][token][32 values], chunks swizzled
    uint16_t B[MX_KS][MX_TN][32];  // weights,     [blk][row][32 values],   chunks swizzled
    float SW[MX_KS][MX_TN];        // weight scales
};
struct MxBias {
    uint16_t X[MX_TM][16];  // [token][8 blocks x (hi, lo)]
    uint16_t W[MX_TN][16];  // [row][8 blocks x (bias, bias)]
};

// Load instructions (64 lanes x 16 B = 1 KB each) of a stage: A, B and the
// scales; the group's last stage (j = 3) also carries the group's Q4 bias
// operands. Wave w issues instructions w, w + 8, ...
template <int DT>
struct MxPlan {
    static constexpr int I_A = MX_KS * MX_TM * 64 / 1024;
    static constexpr int I_B = MX_NW;  // one quant-byte load per wave (Q4: half a wave's lanes)
    static constexpr int I_S = MX_KS * MX_TN * 4 / 1024;
    static constexpr int I_MAIN = I_A + I_B + I_S;
    static constexpr int I_BIAS = DT == 2 ? (int)sizeof(MxBias) / 1024 : 0;
    static_assert(I_A == 4 * MX_NW && I_S == 1, "the issue code below hard-codes this split");
    static_assert(MX_KS * MX_TN * 32 == I_B * 1024, "Q8: a wave's slice is 16 rows x 2 blocks x 32 bytes");
    static_assert(I_BIAS == 0 || I_BIAS == 12, "bias pieces: 8 of X, 4 of W");
    __device__ static int count(int wave, bool last) {
        const int tot = I_MAIN + (last ? I_BIAS : 0);
        return (tot - wave + MX_NW - 1) / MX_NW;
    }
};
static_assert(sizeof(MxStage) * 3 + sizeof(MxBias) <= 160 * 1024, "three stages and the bias operands fit the LDS");

struct MxArgs {
    const uint8_t* qs;    // nncpu's quants, row-major: Q8 32 bytes, Q4 16 bytes per block
    const float* swT;     // [nb + 1][rows_pad] f32 weight scales
    const uint16_t* wbi;  // Q4: [rows_pad][nbp8][2] BF16 biases, twice
    const uint16_t* xb;   // [token tile][nb][256][32] BF16 q_x 2^E (chunks swizzled)
    const uint16_t* xl;   // [xl_tok][nbp8][2] BF16 limbs of X
    float* ws;            // [team * mtiles + mt][2][8 waves][4 tiles][16][64] partial tiles
    float* y;
    size_t y_stride, cols;
    uint32_t qrow;  // bytes per weight row of qs
    int rows, rows_pad, nb, nbp8, ng, n_tok, mtiles, teams, rtiles;
    int rounds;  // whole row tiles per team (data-parallel rounds): team t takes row tiles t, t + teams, ..
    long tail;   // the remaining (rtiles - rounds * teams) row tiles' units, split evenly over the teams
    long tail_q, tail_r;  // tail / teams, tail % teams
};

__device__ __forceinline__ long team_start(long team, long units, int teams) { return team * units / teams; }

// Swizzled position of 16-byte chunk `c` of LDS row `r` (and the inverse:
// the same XOR). A 16-byte read by 16 lanes (rows r .. r + 15, one chunk)
// then covers all 64 banks once: rows r, r + 4, r + 8, r + 12 share a bank
// quarter and take four different positions.
__device__ __forceinline__ int mx_swz(int c, int r) { return c ^ ((r >> 2) & 3); }

// A lane's byte offsets for its loads, fixed for the kernel: each load is a
// uniform (scalar) base plus one of these. The activations are stored tiled
// (xb [token tile][block][256 tokens][32], chunks already swizzled), so each
// 1 KB load is 1 KB of consecutive bytes: wave w's A instructions cover
// token rows 16 w .. 16 w + 15 (a0) and 128 + 16 w .. (a1) of a block; lane
// l's 16 bytes are row l / 4's chunk position l % 4, which holds chunk
// mx_swz(l % 4, row) of the row. The weight quants are read from the split
// layout: wave w's slice is weight rows 16 w .. 16 w + 15 of the stage's two
// blocks, Q8 lane l row 16 w + l / 4, block (l / 2) % 2, bytes 16 (l % 2)
// .. + 15 of it; Q4 lane l < 32 row 16 w + l / 2, block l % 2, all 16
// bytes (brow, the row in the tile; bcol, the byte offset in the row when
// the stage's two blocks are consecutive).
struct MxLane {
    uint32_t a0, a1, bias, sw, brow, bcol;
};

template <int DT>
__device__ __forceinline__ MxLane mx_lane(const MxArgs& g, int wave, int lane) {
    MxLane o;
    o.a0 = (uint32_t)(wave * 1024 + lane * 16);
    o.a1 = (uint32_t)(8192 + wave * 1024 + lane * 16);
    o.bias = (uint32_t)((lane >> 1) * g.nbp8 * 4 + 16 * (lane & 1));
    o.sw = (uint32_t)((lane >> 5) * g.rows_pad * 4 + 16 * (lane & 31));
    if (DT == 1) {
        o.brow = (uint32_t)(16 * wave + (lane >> 2));
        o.bcol = (uint32_t)(16 * (lane & 1) + 32 * ((lane >> 1) & 1));
    } else {
        o.brow = (uint32_t)(16 * wave + ((lane >> 1) & 15));
        o.bcol = (uint32_t)(16 * (lane & 1));
    }
    return o;
}

// One 1 KB direct load (64 lanes x 16 bytes) from base + voff (base
// uniform, in SGPRs) into LDS at dst (uniform; lane l's bytes land at
// dst + 16 l). Issued as asm: for the builtin the compiler cannot tell the
// loads into one stage from the reads of another and drains every load in
// flight before each stage's first LDS read; the waits are explicit instead
// (wait_vm, then a barrier).
__device__ __forceinline__ void lds_load(const void* base, uint32_t voff, void* dst) {
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"((uint32_t)(uintptr_t)dst)
                 : "memory");
}

// Wave w's staging slice of a stage's weight quants: 1 KB at B[1] + 1 KB w,
// inside the BF16 rows 16 w .. 16 w + 15 of block 1 that the wave's own
// conversion writes (so no other wave's slice is overwritten).
__device__ __forceinline__ uint8_t* mx_stage_slice(MxStage& st, int wave) {
    return (uint8_t*)&st.B[1][0][0] + 1024 * wave;
}

// Issue this wave's loads of the stage holding blocks 2 j, 2 j + 1 of group
// gi of row tile rt. Blocks past nb are clamped to the last block (never
// computed); tokens and X limbs are padded to whole tiles with zeros, weight
// rows past the matrix read its last row (their scales are zero and their
// outputs are never stored); the scale table has a spare block row past nb.
template <int DT>
__device__ __forceinline__ void mx_issue(MxStage& st, MxBias& bias, const MxArgs& g, const MxLane& o, int rt, int gi,
                                         int j, int wave, int m0) {
    const int n0 = rt * MX_TN;
    const int b0 = gi * MX_GRP + j * MX_KS;
    const int bA = b0 < g.nb ? b0 : g.nb - 1, bB = b0 + 1 < g.nb ? b0 + 1 : g.nb - 1;
    const uint8_t* xb = (const uint8_t*)g.xb + (size_t)(m0 / MX_TM) * g.nb * (MX_TM * 64);
    uint8_t* A = (uint8_t*)&st.A[0][0][0];
    lds_load(xb + (size_t)bA * (MX_TM * 64), o.a0, A + wave * 1024);
    lds_load(xb + (size_t)bA * (MX_TM * 64), o.a1, A + (wave + 8) * 1024);
    lds_load(xb + (size_t)bB * (MX_TM * 64), o.a0, A + (wave + 16) * 1024);
    lds_load(xb + (size_t)bB * (MX_TM * 64), o.a1, A + (wave + 24) * 1024);
    {
        constexpr int BLK = DT == 1 ? 32 : 16;  // quant bytes per block
        const uint8_t* wq = g.qs + (size_t)n0 * g.qrow + (size_t)bA * BLK;
        const int last = g.rows - 1 - n0;  // rows past the matrix read its last row
        const uint32_t r = (int)o.brow < last ? o.brow : (uint32_t)last;
        // bB == bA when the second block is past nb: both halves then read bA.
        const uint32_t col = bB > bA ? o.bcol : (DT == 1 ? (o.bcol & 16u) : 0u);
        const uint32_t voff = r * g.qrow + col;
        if (DT == 1 || (__lane_id() < 32)) lds_load(wq, voff, mx_stage_slice(st, wave));
    }
    if (wave == 0) lds_load((const uint8_t*)g.swT + ((size_t)bA * g.rows_pad + n0) * 4, o.sw, &st.SW[0][0]);
    if (DT == 2 && j == 3) {
        // Bias pieces 0..11 are instructions 41..52: waves 1..7 take pieces
        // 0..6, waves 0..4 pieces 7..11. Piece p < 8: X of tokens 32 p ..,
        // else the biases of rows 32 (p - 8) ..
        const uint8_t* xl = (const uint8_t*)g.xl + ((size_t)m0 * g.nbp8 + (size_t)gi * MX_GRP) * 4;
        const uint8_t* wi = (const uint8_t*)g.wbi + ((size_t)n0 * g.nbp8 + (size_t)gi * MX_GRP) * 4;
        const size_t rows32 = (size_t)32 * g.nbp8 * 4;
        uint8_t* X = (uint8_t*)&bias.X[0][0];
        uint8_t* W = (uint8_t*)&bias.W[0][0];
        if (wave >= 1) lds_load(xl + (wave - 1) * rows32, o.bias, X + (wave - 1) * 1024);
        if (wave == 0) lds_load(xl + 7 * rows32, o.bias, X + 7 * 1024);
        if (wave >= 1 && wave <= 4) lds_load(wi + (wave - 1) * rows32, o.bias, W + (wave - 1) * 1024);
    }
}

// s_waitcnt vmcnt(n) for a wave-uniform n (the immediate must be a constant).
__device__ __forceinline__ void wait_vm(int n) {
    switch (n) {
#define NNH_W(k) case k: __builtin_amdgcn_s_waitcnt(NNH_VMCNT(k)); break;
        NNH_W(0) NNH_W(1) NNH_W(2) NNH_W(3) NNH_W(4) NNH_W(5) NNH_W(6) NNH_W(7) NNH_W(8) NNH_W(9)
        NNH_W(10) NNH_W(11) NNH_W(12) NNH_W(13) NNH_W(14) NNH_W(15) NNH_W(16) NNH_W(17) NNH_W(18) NNH_W(19)
#undef NNH_W
        default: __builtin_amdgcn_s_waitcnt(NNH_VMCNT(0)); break;
    }
}

// The high halves of two f32 values (exact BF16 values) as one BF16 pair.
__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// This wave's staged quants of the stage to BF16 operand rows (exact: Q8
// -127..127 and Q4 0..15 are small integers), written into rows
// 16 wave .. + 15 of both blocks, chunks swizzled as the reads expect. The
// slice is read before any of it is overwritten (each lane's writes depend
// on its read, and the slice lies inside the rows the wave writes).
template <int DT>
__device__ __forceinline__ void mx_convert(MxStage& st, int wave, int lane) {
    const int row = 16 * wave + (lane >> 2), bsel = (lane >> 1) & 1;
    uint16_t* dst = &st.B[bsel][row][0];
    uint32_t o[8];
    int c0, c1;
    if (DT == 1) {
        // 16 signed quants: elements 16 (lane % 2) .. + 15 of the block.
        const int4 v = *(const int4*)(mx_stage_slice(st, wave) + 16 * lane);
        const int w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            o[2 * d] = bf16_pair((float)(int8_t)w[d], (float)(int8_t)(w[d] >> 8));
            o[2 * d + 1] = bf16_pair((float)(int8_t)(w[d] >> 16), (float)(w[d] >> 24));
        }
        c0 = 2 * (lane & 1);
        c1 = c0 + 1;
    } else {
        // 8 bytes of the block: elements 8 p .. 8 p + 7 in the low nibbles,
        // 16 + 8 p .. in the high ones (nncpu's order), p = lane % 2.
        const uint2 v = *(const uint2*)(mx_stage_slice(st, wave) + 8 * lane);
        const uint32_t w[4] = {v.x & 0x0F0F0F0Fu, v.y & 0x0F0F0F0Fu, (v.x >> 4) & 0x0F0F0F0Fu,
                               (v.y >> 4) & 0x0F0F0F0Fu};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            o[2 * d] = bf16_pair((float)(w[d] & 255u), (float)((w[d] >> 8) & 255u));
            o[2 * d + 1] = bf16_pair((float)((w[d] >> 16) & 255u), (float)(w[d] >> 24));
        }
        c0 = lane & 1;
        c1 = c0 + 2;
    }
    *(uint4*)(dst + 8 * mx_swz(c0, row)) = make_uint4(o[0], o[1], o[2], o[3]);
    *(uint4*)(dst + 8 * mx_swz(c1, row)) = make_uint4(o[4], o[5], o[6], o[7]);
}

__device__ __forceinline__ v8bf lds_bf8(const uint16_t* row, int chunk, int r) {
    return __builtin_bit_cast(v8bf, *(const int4*)(row + 8 * mx_swz(chunk, r)));
}

typedef v16f MxTiles[2][2];  // [token tile][row tile]

// One stage's blocks for the wave's 2 x 2 tiles: lane (c, h) holds weight
// rows rw + c, rw + 32 + c and, per MFMA, 8 K values of token rows rm + c,
// rm + 32 + c. The two MFMAs of a block take chunks (2h) and (2h + 1) of the
// 4 in a row, the same for both operands, so the pair covers the block's 32
// values.
__device__ __forceinline__ void mx_compute(const MxStage& st, int nblk, int rw, int rm, int c, int h, MxTiles& acc) {
#pragma unroll
    for (int j = 0; j < MX_KS; ++j) {
        if (j >= nblk) break;
        float sw[2];
        v8bf Bv[2][2], Av[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int rb = rw + 32 * i + c, ra = rm + 32 * i + c;
            sw[i] = st.SW[j][rb];
            Bv[i][0] = lds_bf8(&st.B[j][rb][0], 2 * h, rb);
            Bv[i][1] = lds_bf8(&st.B[j][rb][0], 2 * h + 1, rb);
            Av[i][0] = lds_bf8(&st.A[j][ra][0], 2 * h, ra);
            Av[i][1] = lds_bf8(&st.A[j][ra][0], 2 * h + 1, ra);
        }
        // Two result sets in turn, so the FMAs of one tile run while the
        // matrix unit forms the next: tiles (0,0), (0,1), (1,0), (1,1).
        const v16f z = {};
        v16f P0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Av[0][0], Bv[0][0], z, 0, 0, 0);
        P0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Av[0][1], Bv[0][1], P0, 0, 0, 0);
        v16f P1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Av[0][0], Bv[1][0], z, 0, 0, 0);
        P1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Av[0][1], Bv[1][1], P1, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[0][0][r] = __builtin_fmaf(P0[r], sw[0], acc[0][0][r]);
        P0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Av[1][0], Bv[0][0], z, 0, 0, 0);
        P0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Av[1][1], Bv[0][1], P0, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[0][1][r] = __builtin_fmaf(P1[r], sw[1], acc[0][1][r]);
        P1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Av[1][0], Bv[1][0], z, 0, 0, 0);
        P1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Av[1][1], Bv[1][1], P1, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[1][0][r] = __builtin_fmaf(P0[r], sw[0], acc[1][0][r]);
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[1][1][r] = __builtin_fmaf(P1[r], sw[1], acc[1][1][r]);
    }
}

// End of a tile segment: the totals to y (whole tile) or to the workspace
// slot (partial tile). Result register r of lane (c, h) in tile (ti, ri) is
// token rm + 32 ti + 8 (r / 4) + 4 h + r % 4, weight row rw + 32 ri + c.
__device__ __forceinline__ void mx_store(const MxArgs& g, MxTiles& tot, bool whole, int slot, int lid, int wave,
                                         int lane, int n0, int m0, int rw, int rm, int c, int h) {
    // The stride and bases pass through an empty asm: without it the
    // compiler hoists the loop-invariant row addresses out of the K loop
    // and holds them in VGPRs for its whole length.
    if (whole) {
        size_t ys = g.y_stride;
        asm volatile("" : "+s"(ys));
        const int mb = m0 + rm + 4 * h;
        float* yb = g.y + (size_t)mb * ys + n0 + rw + c;
#pragma unroll
        for (int ri = 0; ri < 2; ++ri) {
            if (n0 + rw + 32 * ri + c >= g.rows) continue;
#pragma unroll
            for (int ti = 0; ti < 2; ++ti)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int dm = 32 * ti + 8 * (r >> 2) + (r & 3);
                    if (mb + dm < g.n_tok) yb[(size_t)dm * ys + 32 * ri] = tot[ti][ri][r];
                }
        }
    } else {
        size_t off = (((size_t)lid * 2 + slot) * MX_NW + wave) * 4096 + lane;
        asm volatile("" : "+v"(off));
        float* p = g.ws + off;
#pragma unroll
        for (int ti = 0; ti < 2; ++ti)
#pragma unroll
            for (int ri = 0; ri < 2; ++ri)
#pragma unroll
                for (int r = 0; r < 16; ++r) p[((ti * 2 + ri) * 16 + r) * 64] = tot[ti][ri][r];
    }
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int ri = 0; ri < 2; ++ri)
#pragma unroll
            for (int r = 0; r < 16; ++r) tot[ti][ri][r] = 0.0f;
}

// A team's units: its data-parallel row tiles (team, team + teams, .., each
// over all its groups), then its share of the tail, a contiguous range of
// the remaining row tiles' units that may start and end inside a tile.
struct MxCursor {
    int k, rt, gi;  // unit index within the team's work, its row tile and group
};

struct MxLoop {
    int nst;           // stages: 4 per unit
    int nk, dp;        // the team's units, of them data-parallel
    int trt, tgi;      // the first tail unit's row tile and group
    MxCursor cc, ic;   // compute cursor (the stage being computed), issue cursor (the stage being issued)
    int seg_k0, seg_gi0;  // unit index and group the current segment began at
    int lid, wave, lane, c, h, rw, rm, m0;
    int chunk;         // groups in the current f32 chunk
    MxLane o;
};

__device__ __forceinline__ void mx_advance(MxCursor& c, const MxLoop& L, const MxArgs& g) {
    ++c.k;
    ++c.gi;
    if (c.k == L.dp) {  // the data-parallel tiles are done: the tail share
        c.rt = L.trt;
        c.gi = L.tgi;
    } else if (c.gi == g.ng) {
        c.gi = 0;
        c.rt += c.k < L.dp ? g.teams : 1;
    }
}

// One step of the ring of three buffers: stage s (J = s % 4) is in `cur`;
// stage s + 2 goes into `nxt`, the buffer stage s - 1 was computed from.
template <int DT, int J>
__device__ __forceinline__ void mx_step(MxStage& cur, MxStage& nxt, MxBias& bias, const MxArgs& g, MxLoop& L, int s,
                                        MxTiles& acc, MxTiles& tot) {
    using P = MxPlan<DT>;
    if (s >= L.nst) return;
    // This wave's loads of stage s are done once at most those of s + 1 are
    // outstanding (vmcnt counts down in issue order).
    wait_vm(s + 1 < L.nst ? P::count(L.wave, ((J + 1) & 3) == 3) : 0);
    asm volatile("" ::: "memory");
    mx_convert<DT>(cur, L.wave, L.lane);
    // Every wave's loads of stage s have landed, its quants are converted,
    // and every wave is done with stage s - 1 (the wave's own LDS writes
    // first, then a bare barrier: __syncthreads would also wait for the
    // loads still in flight; the memory clobber keeps the LDS reads after it).
    __builtin_amdgcn_s_waitcnt(NNH_LGKMCNT0);
    asm volatile("s_barrier" ::: "memory");
    if (s + 2 < L.nst) {
        if (J == 2) mx_advance(L.ic, L, g);  // stage s + 2 opens the next group
        mx_issue<DT>(nxt, bias, g, L.o, L.ic.rt, L.ic.gi, (J + 2) & 3, L.wave, L.m0);
    }
    const int nblk = g.nb - (L.cc.gi * MX_GRP + J * MX_KS);
    mx_compute(cur, nblk, L.rw, L.rm, L.c, L.h, acc);
    if (J != 3) return;
    if (DT == 2) {
        // sum over the group's 8 blocks of bias[n,b] (hi + lo)[m,b]: lane half
        // h supplies blocks 4h .. 4h + 3, two limbs each.
#pragma unroll
        for (int ti = 0; ti < 2; ++ti) {
            const v8bf X = __builtin_bit_cast(v8bf, *(const int4*)&bias.X[L.rm + 32 * ti + L.c][8 * L.h]);
#pragma unroll
            for (int ri = 0; ri < 2; ++ri) {
                const v8bf W = __builtin_bit_cast(v8bf, *(const int4*)&bias.W[L.rw + 32 * ri + L.c][8 * L.h]);
                acc[ti][ri] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(X, W, acc[ti][ri], 0, 0, 0);
            }
        }
    }
    const bool seg_end = s + 1 == L.nst || L.cc.gi + 1 == g.ng;
    if (++L.chunk == MX_FOLD_GROUPS || seg_end) {
#pragma unroll
        for (int ti = 0; ti < 2; ++ti)
#pragma unroll
            for (int ri = 0; ri < 2; ++ri)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    tot[ti][ri][r] += acc[ti][ri][r];
                    acc[ti][ri][r] = 0.0f;
                }
        L.chunk = 0;
    }
    if (seg_end) {
        // The segment is whole iff it spans its tile's groups; a partial one
        // is the team's first tail segment (slot 0) or its last (slot 1).
        const bool whole = L.seg_gi0 == 0 && L.cc.gi + 1 == g.ng;
        mx_store(g, tot, whole, L.seg_k0 == L.dp ? 0 : 1, L.lid, L.wave, L.lane, L.cc.rt * MX_TN, L.m0, L.rw, L.rm,
                 L.c, L.h);
    }
    mx_advance(L.cc, L, g);
    if (seg_end) {
        L.seg_k0 = L.cc.k;
        L.seg_gi0 = L.cc.gi;
    }
}

template <int DT>
__global__ __launch_bounds__(MX_NW * 64) void gemm_mx_kernel(MxArgs g) {
    // Three distinct objects, not one array: the compiler then sees that the
    // loads into one stage do not alias the reads of another.
    __shared__ __attribute__((aligned(16))) MxStage s0, s1, s2;
    __shared__ __attribute__((aligned(16))) MxBias bias;
    const int tid = threadIdx.x;
    MxLoop L;
    L.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    L.lane = tid & 63;
    L.h = L.lane >> 5;
    L.c = L.lane & 31;
    L.rw = (L.wave & 1) * 64;   // rows
    L.rm = (L.wave >> 1) * 64;  // tokens
    // Workgroups go round-robin to the 8 XCDs; renumber them so each XCD
    // runs a contiguous range of logical ids, i.e. whole teams.
    const int total = gridDim.x, per = total / 8, rem = total % 8;
    const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
    L.lid = xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
    const int team = L.lid / g.mtiles, mt = L.lid - team * g.mtiles;
    L.m0 = mt * MX_TM;
    const long t0 = team_start(team, g.tail, g.teams), t1 = team_start(team + 1, g.tail, g.teams);
    const long ut = (long)g.rounds * g.teams * g.ng + t0;  // the first tail unit
    L.dp = g.rounds * g.ng;
    L.nk = L.dp + (int)(t1 - t0);
    L.nst = L.nk * MX_NS;
    L.trt = (int)(ut / g.ng);
    L.tgi = (int)(ut - (long)L.trt * g.ng);
    L.cc.k = 0;
    L.cc.rt = L.dp > 0 ? team : L.trt;
    L.cc.gi = L.dp > 0 ? 0 : L.tgi;
    L.ic = L.cc;
    L.seg_k0 = 0;
    L.seg_gi0 = L.cc.gi;
    L.chunk = 0;
    L.o = mx_lane<DT>(g, L.wave, L.lane);

    MxTiles tot, acc;
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int ri = 0; ri < 2; ++ri)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                tot[ti][ri][r] = 0.0f;
                acc[ti][ri][r] = 0.0f;
            }

    // Stages 0 and 1 (the first group's blocks 0..3), then the ring: step
    // k of 12 computes buffer k % 3 and refills buffer (k + 2) % 3.
    mx_issue<DT>(s0, bias, g, L.o, L.ic.rt, L.ic.gi, 0, L.wave, L.m0);
    mx_issue<DT>(s1, bias, g, L.o, L.ic.rt, L.ic.gi, 1, L.wave, L.m0);
    for (int s = 0; s < L.nst; s += 12) {
        mx_step<DT, 0>(s0, s2, bias, g, L, s, acc, tot);
        mx_step<DT, 1>(s1, s0, bias, g, L, s + 1, acc, tot);
        mx_step<DT, 2>(s2, s1, bias, g, L, s + 2, acc, tot);
        mx_step<DT, 3>(s0, s2, bias, g, L, s + 3, acc, tot);
        mx_step<DT, 0>(s1, s0, bias, g, L, s + 4, acc, tot);
        mx_step<DT, 1>(s2, s1, bias, g, L, s + 5, acc, tot);
        mx_step<DT, 2>(s0, s2, bias, g, L, s + 6, acc, tot);
        mx_step<DT, 3>(s1, s0, bias, g, L, s + 7, acc, tot);
        mx_step<DT, 0>(s2, s1, bias, g, L, s + 8, acc, tot);
        mx_step<DT, 1>(s0, s2, bias, g, L, s + 9, acc, tot);
        mx_step<DT, 2>(s1, s0, bias, g, L, s + 10, acc, tot);
        mx_step<DT, 3>(s2, s1, bias, g, L, s + 11, acc, tot);
    }
}

// The team whose range holds unit u.
__device__ __forceinline__ int team_of(long u, long units, int teams) {
    int t = (int)(u * teams / units);
    while (t + 1 < teams && team_start(t + 1, units, teams) <= u) ++t;
    while (t > 0 && team_start(t, units, teams) > u) --t;
    return t;
}

// y of every tail tile split between teams = its partial tiles added in
// team order, in f64, rounded once. One workgroup of 256 threads per (tail
// tile, wave region); thread (tt, lane) takes MFMA tile tt = 2 ti + ri of
// that wave's region, 16 results. Whole tiles exit at once.
__global__ __launch_bounds__(256) void gemm_mx_fixup_kernel(MxArgs g) {
    const int tile = blockIdx.x / MX_NW, wave = blockIdx.x % MX_NW;
    const int tr = tile / g.mtiles, mt = tile - tr * g.mtiles;
    const int rt = g.rounds * g.teams + tr;
    const long ua = (long)tr * g.ng, ub = ua + g.ng;  // tail units of the tile
    const int t0 = team_of(ua, g.tail, g.teams), t1 = team_of(ub - 1, g.tail, g.teams);
    if (t0 == t1) return;
    const int lane = threadIdx.x & 63, tt = threadIdx.x >> 6;
    const int ti = tt >> 1, ri = tt & 1, h = lane >> 5, c = lane & 31;
    const int rw = (wave & 1) * 64, rm = (wave >> 1) * 64;
    double sum[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) sum[r] = 0.0;
    // Partials are loaded 8 teams at a time before any is added (one round
    // trip per 8, not per team), then added in team order. The teams' tail
    // starts team_start(tm) = floor(tm tail / teams) are walked by quotient
    // and remainder (no division per team).
    constexpr int BATCH = 8;
    long ts = team_start(t0, g.tail, g.teams);
    long rem = (long)t0 * g.tail - ts * g.teams;
    for (int tb = t0; tb <= t1; tb += BATCH) {
        float v[BATCH][16];
#pragma unroll
        for (int i = 0; i < BATCH; ++i) {
            const int tm = tb + i;
            long te = ts + g.tail_q;
            long rn = rem + g.tail_r;
            if (rn >= g.teams) {
                ++te;
                rn -= g.teams;
            }
            // Teams past t1 and empty tail shares (tail < teams) contribute
            // nothing: they load team t0's slot (a valid address, so the
            // load needs no branch) and the value is dropped by a select.
            const bool use = tm <= t1 && te > ts;
            const int slot = use && ts < ua ? 1 : 0;
            const float* p = g.ws + (((size_t)(use ? tm : t0) * g.mtiles + mt) * 2 + (use ? slot : 0)) * MX_NW * 4096 +
                             (size_t)wave * 4096 + (size_t)tt * 1024 + lane;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float x = p[r * 64];
                v[i][r] = use ? x : 0.0f;
            }
            ts = te;
            rem = rn;
        }
#pragma unroll
        for (int i = 0; i < BATCH; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) sum[r] += (double)v[i][r];
    }
    const int n = rt * MX_TN + rw + 32 * ri + c;
    if (n >= g.rows) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int m = mt * MX_TM + rm + 32 * ti + 8 * (r >> 2) + 4 * h + (r & 3);
        if (m < g.n_tok) g.y[(size_t)m * g.y_stride + n] = (float)sum[r];
    }
}

struct MxSched {
    int mtiles, rtiles, ng, teams, rounds;
    long units, tail;
};

MxSched mx_sched(int rows, int nb, int n_tok) {
    MxSched s;
    s.mtiles = ceil_div(n_tok, MX_TM);
    s.rtiles = ceil_div(rows, MX_TN);
    s.ng = ceil_div(nb, MX_GRP);
    s.units = (long)s.rtiles * s.ng;
    long teams = cu_count() / s.mtiles;
    const long most = s.units / MX_MIN_UNITS;
    if (teams > most) teams = most;
    s.teams = teams < 1 ? 1 : (int)teams;
    s.rounds = s.rtiles / s.teams;
    s.tail = (long)(s.rtiles - s.rounds * s.teams) * s.ng;
    return s;
}

}  // namespace

int mx_nbp8(int nb) { return ceil_div(nb, MX_GRP) * MX_GRP; }
int mx_xl_tok(int n_tok) { return ceil_div(n_tok, MX_TM) * MX_TM; }

void launch_quantize_mx(const float* x, size_t x_stride, int cols, int n_tok, int8_t* q, uint16_t* s, double* sx,
                        float* sxT, int tok_pad, uint16_t* xb, uint16_t* xl, hipStream_t st) {
    const int nbp8 = mx_nbp8(cols / 32), xl_tok = mx_xl_tok(n_tok);
    const long blocks = (long)nbp8 * xl_tok;
    quantize_mx_kernel<<<ceil_div(blocks, 8), 256, 0, st>>>(x, x_stride, cols, n_tok, nbp8, q, s, sx, sxT, tok_pad,
                                                            xl_tok, xb, xl);
}

size_t mx_bias_bytes(int rows, int nb) { return (size_t)gemm_rows_pad(rows) * mx_nbp8(nb) * 4; }
size_t mx_xl_bytes(int n_tok, int nb) { return (size_t)mx_xl_tok(n_tok) * mx_nbp8(nb) * 4; }

void launch_mx_bias(const uint16_t* bi, int rows, int nb, uint16_t* wbi, hipStream_t st) {
    const int rp = gemm_rows_pad(rows);
    const size_t m = (size_t)rp * mx_nbp8(nb);
    mx_bias_kernel<<<(unsigned)((m + 255) / 256), 256, 0, st>>>(bi, wbi, rows, rp, nb, mx_nbp8(nb));
}

size_t gemm_mx_workspace_bytes(int rows, int nb, int n_tok) {
    const MxSched s = mx_sched(rows, nb, n_tok);
    return (size_t)s.teams * s.mtiles * 2 * MX_TM * MX_TN * sizeof(float);
}

void launch_gemm_mx(int dtype, const uint8_t* qs, const float* swT, const uint16_t* wbi, const uint16_t* xb,
                    const uint16_t* xl, int rows, int nb, int n_tok, float* y, size_t y_stride, float* ws,
                    hipStream_t st) {
    const MxSched s = mx_sched(rows, nb, n_tok);
    MxArgs g;
    g.qs = qs;
    g.qrow = (uint32_t)(dtype == 1 ? (size_t)nb * 32 : (size_t)nb * 16);
    g.swT = swT;
    g.wbi = wbi;
    g.xb = xb;
    g.xl = xl;
    g.ws = ws;
    g.y = y;
    g.y_stride = y_stride;
    g.cols = (size_t)nb * 32;
    g.rows = rows;
    g.rows_pad = gemm_rows_pad(rows);
    g.nb = nb;
    g.nbp8 = mx_nbp8(nb);
    g.ng = s.ng;
    g.n_tok = n_tok;
    g.mtiles = s.mtiles;
    g.teams = s.teams;
    g.rtiles = s.rtiles;
    g.rounds = s.rounds;
    g.tail = s.tail;
    g.tail_q = s.tail / s.teams;
    g.tail_r = s.tail % s.teams;
    const dim3 grid(s.teams * s.mtiles), block(MX_NW * 64);
    if (dtype == 1)
        gemm_mx_kernel<1><<<grid, block, 0, st>>>(g);
    else
        gemm_mx_kernel<2><<<grid, block, 0, st>>>(g);
    // A tail tile is split iff some team's tail share starts inside it.
    bool split = false;
    for (long t = 1; t < s.teams && !split; ++t) split = (t * s.tail / s.teams) % s.ng != 0;
    const int tail_tiles = s.rtiles - s.rounds * s.teams;
    if (split) gemm_mx_fixup_kernel<<<tail_tiles * s.mtiles * MX_NW, 256, 0, st>>>(g);
}

}  // namespace nnh
