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
// Epilogue per block and output: acc = fma(P, s_w * s_x, acc) (+ Q4
// acc = fma(bias, s_x * sum q_x, acc)); P and the scale products are exact.
// The accumulator is f64 (an f32 form is built for short rows; an f32 sum
// over K = 18944 would take most of the 1e-5 tolerance next to nncpu's own
// f32 rounding). nncpu's per-32 BF16 scales make this epilogue, not the
// MFMA, the compute bound: 3 (Q8) / 4 (Q4) VALU ops per output and block
// against 32 MACs.
//
// Workgroup: 128 weight rows x 128 tokens, 4 waves as 2 x 2, each wave a
// 64 x 64 block of 2 x 2 MFMA tiles. A chunk of KB blocks of both operands
// and their scales (as f32) is staged in LDS, double-buffered, while the
// previous chunk is computed; the small footprint lets several workgroups
// share a CU and hide each other's latency.

#include "common.h"

namespace nnh {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

template <int DT, int KB, typename ACC>
__global__ __launch_bounds__(256) void gemm_i8_kernel(const uint8_t* __restrict__ qs, const uint16_t* __restrict__ sc,
                                                      const uint16_t* __restrict__ bi, const int8_t* __restrict__ aq,
                                                      const double* __restrict__ asx, int rows, int nb, int n_tok,
                                                      float* __restrict__ y, size_t y_stride) {
    constexpr int QB = DT == 1 ? 32 : 16;  // weight bytes per row and block
    __shared__ __attribute__((aligned(16))) uint8_t sA[2][KB][128 * QB];
    __shared__ __attribute__((aligned(16))) int8_t sB[2][KB][128 * 32];
    __shared__ float sSW[2][KB][128];
    __shared__ float sBI[DT == 2 ? 2 : 1][DT == 2 ? KB : 1][128];
    __shared__ float2 sSX[2][KB][128];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, l = tid & 63;
    const int h = l >> 5, c = l & 31;
    const int wn = wave >> 1, wm = wave & 1;  // 64-row, 64-token quadrant of the tile
    const int n0 = blockIdx.y * 128;
    const int m0 = blockIdx.x * 128;
    const size_t cols = (size_t)nb * 32;
    const size_t qrow = DT == 1 ? cols : cols / 2;

    constexpr int A_PER = 128 * KB * QB / 16 / 256;  // 16-byte pieces per thread and chunk
    constexpr int B_PER = 128 * KB * 32 / 16 / 256;
    constexpr int S_PER = 128 * KB / 256;
    static_assert(A_PER >= 1 && B_PER >= 1 && S_PER >= 1, "KB too small");

    int4 ra[A_PER], rb[B_PER];
    uint32_t rsw[S_PER], rbi[S_PER];
    float2 rsx[S_PER];

    auto gload = [&](int b0) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int p = tid + 256 * i;
            constexpr int per_row = KB * QB / 16;
            const int row = p / per_row, part = p - row * per_row;
            const int n = n0 + row < rows ? n0 + row : rows - 1;
            const int blk = (part * 16) / QB;
            const size_t b = b0 + blk < nb ? b0 + blk : nb - 1;
            ra[i] = load_nt16(qs + (size_t)n * qrow + b * QB + (part * 16) % QB);
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int p = tid + 256 * i;
            constexpr int per_row = KB * 2;
            const int row = p / per_row, part = p - row * per_row;
            const int m = m0 + row < n_tok ? m0 + row : n_tok - 1;
            const size_t b = b0 + (part >> 1) < nb ? b0 + (part >> 1) : nb - 1;
            rb[i] = *(const int4*)(aq + (size_t)m * cols + 32 * b + 16 * (part & 1));
        }
#pragma unroll
        for (int i = 0; i < S_PER; ++i) {
            const int p = tid + 256 * i;
            const int blk = p / 128, row = p - blk * 128;
            const bool bok = b0 + blk < nb;
            const size_t b = bok ? b0 + blk : nb - 1;
            const bool nok = bok && n0 + row < rows;
            const int n = n0 + row < rows ? n0 + row : rows - 1;
            const int m = m0 + row < n_tok ? m0 + row : n_tok - 1;
            rsw[i] = nok ? sc[(size_t)n * nb + b] : 0u;
            if (DT == 2) rbi[i] = nok ? bi[(size_t)n * nb + b] : 0u;
            const double2 v = ((const double2*)asx)[(size_t)m * nb + b];
            rsx[i] = make_float2((float)v.x, (float)v.y);  // both exact in f32
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int p = tid + 256 * i;
            constexpr int per_row = KB * QB / 16;
            const int row = p / per_row, part = p - row * per_row;
            *(int4*)&sA[buf][(part * 16) / QB][row * QB + (part * 16) % QB] = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int p = tid + 256 * i;
            constexpr int per_row = KB * 2;
            const int row = p / per_row, part = p - row * per_row;
            *(int4*)&sB[buf][part >> 1][row * 32 + 16 * (part & 1)] = rb[i];
        }
#pragma unroll
        for (int i = 0; i < S_PER; ++i) {
            const int p = tid + 256 * i;
            const int blk = p / 128, row = p - blk * 128;
            sSW[buf][blk][row] = bf16f(rsw[i]);
            if (DT == 2) sBI[buf][blk][row] = bf16f(rbi[i]);
            sSX[buf][blk][row] = rsx[i];
        }
    };

    ACC acc[2][2][16];  // [A tile][B tile][register]
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][t][r] = 0;

    gload(0);
    lstore(0);
    __syncthreads();
    int buf = 0;
    for (int b0 = 0; b0 < nb; b0 += KB) {
        const bool more = b0 + KB < nb;
        if (more) gload(b0 + KB);
        const int kb_end = nb - b0 < KB ? nb - b0 : KB;
        for (int j = 0; j < kb_end; ++j) {
            v4i av[2];
            float sw[2][16];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int rowA = wn * 64 + i * 32;
                int4 a;
                if (DT == 1) {
                    a = *(const int4*)&sA[buf][j][(rowA + c) * 32 + 16 * h];
                } else {
                    const int4 q = *(const int4*)&sA[buf][j][(rowA + c) * 16];
                    const int sh = 4 * h, mk = 0x0f0f0f0f;
                    a.x = (int)((unsigned)q.x >> sh) & mk;
                    a.y = (int)((unsigned)q.y >> sh) & mk;
                    a.z = (int)((unsigned)q.z >> sh) & mk;
                    a.w = (int)((unsigned)q.w >> sh) & mk;
                }
                av[i] = v4i{a.x, a.y, a.z, a.w};
                const float* swp = &sSW[buf][j][rowA + 4 * h];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float4 v = *(const float4*)(swp + 8 * g);
                    sw[i][4 * g] = v.x;
                    sw[i][4 * g + 1] = v.y;
                    sw[i][4 * g + 2] = v.z;
                    sw[i][4 * g + 3] = v.w;
                }
            }
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int colB = wm * 64 + t * 32;
                const int4 bq = *(const int4*)&sB[buf][j][(colB + c) * 32 + 16 * h];
                const v4i bv = {bq.x, bq.y, bq.z, bq.w};
                const float2 sx = sSX[buf][j][colB + c];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    v16i z = {};
                    const v16i P = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv, z, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const float s = sw[i][r] * sx.x;  // exact: 8 x 8 significant bits
                        if (sizeof(ACC) == 4)
                            acc[i][t][r] = __builtin_fmaf((float)P[r], s, (float)acc[i][t][r]);
                        else
                            acc[i][t][r] = __builtin_fma((double)P[r], (double)s, (double)acc[i][t][r]);
                    }
                    if (DT == 2) {
                        const float* bip = &sBI[buf][j][wn * 64 + i * 32 + 4 * h];
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            const float4 v = *(const float4*)(bip + 8 * g);
                            const float bw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                if (sizeof(ACC) == 4)
                                    acc[i][t][4 * g + q] = __builtin_fmaf(bw[q], sx.y, (float)acc[i][t][4 * g + q]);
                                else
                                    acc[i][t][4 * g + q] =
                                        __builtin_fma((double)bw[q], (double)sx.y, (double)acc[i][t][4 * g + q]);
                            }
                        }
                    }
                }
            }
        }
        if (more) {
            __syncthreads();  // every wave is done reading buf ^ 1 from the chunk before
            lstore(buf ^ 1);
            __syncthreads();
            buf ^= 1;
        }
    }

#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int m = m0 + wm * 64 + t * 32 + c;
        if (m >= n_tok) continue;
        float* yr = y + (size_t)m * y_stride;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int n = n0 + wn * 64 + i * 32 + (r / 4) * 8 + 4 * h + (r % 4);
                if (n < rows) yr[n] = (float)acc[i][t][r];
            }
    }
}

}  // namespace

// The f32 accumulator is used from this many blocks down: none for now,
// f64 keeps every output within one f32 ulp of the exact sum, which the
// tests use to pin each MFMA block dot.
constexpr int GEMM_F64_MIN_NB = 0;

void launch_gemm_i8(int dtype, const uint8_t* qs, const uint16_t* scales, const uint16_t* biases, const int8_t* aq,
                    const double* asx, int rows, int nb, int n_tok, float* y, size_t y_stride, hipStream_t st) {
    dim3 grid(ceil_div(n_tok, 128), ceil_div(rows, 128)), block(256);
    const bool wide = nb > GEMM_F64_MIN_NB;
#define NNH_G(DT, ACC) gemm_i8_kernel<DT, 2, ACC><<<grid, block, 0, st>>>(qs, scales, biases, aq, asx, rows, nb, n_tok, y, y_stride)
    if (dtype == 1) {
        if (wide) NNH_G(1, double); else NNH_G(1, float);
    } else {
        if (wide) NNH_G(2, double); else NNH_G(2, float);
    }
#undef NNH_G
}

}  // namespace nnh
