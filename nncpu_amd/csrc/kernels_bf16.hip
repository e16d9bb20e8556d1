// The BF16 weight format (DType::BF16, WeightFormat::Bf16; the loader also
// keeps any matrix whose rows are not whole 32-element blocks in it,
// crates/nncpu/src/model/load.rs:302-303), bit-exact against nncpu's
// kernels (crates/nncpu/src/kernels/mod.rs:337-406, 454-485; scalar.rs:555-628;
// avx2.rs:1144-1234):
//
//   cols % 8 != 0            gemv_bf16_f64 (mod.rs:556-564): per row, f64
//                            products summed in order, rounded once.
//   rows % 4 == 0            the 4-row kernel: per row 8 FMA chains (chain l
//                            over elements 8i + l, i in order), reduced
//                            ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)) (the hadd tree).
//   else, cols % 32 == 0     the 1-row kernel with four accumulators: 32
//                            chains (chain 8j + l over elements 32i + 8j + l),
//                            v[l] = (a_l + a_{8+l}) + (a_{16+l} + a_{24+l}), hsum8(v).
//   else                     the 1-row kernel with one accumulator: 8 chains,
//                            hsum8.
//
// A batch gives every vector the single-vector bits (mod.rs:454-485 runs the
// 4-row kernel per token or repeats the single gemv).
//
// Device layout for the chain paths (built at upload): a row's steps in
// blocks of 8, each chain's 8 steps of a block in one 16-byte piece, and the
// rows in groups of 64 / C (the rows of one wave) stored block by block, so a
// lane running chain c reads 16 contiguous bytes per 8 steps and a wave reads
// 1 KB of consecutive bytes per block. x is staged in LDS transposed the same
// way (xt[c][i] = x[i C + c]), so a lane's 8 x values of a block are two
// 16-byte reads; up to 4 vectors share each weight load. A chain's steps are
// one lane's FMA sequence in order, so the parallelism is rows x C lanes: a
// wave reads the x values of a whole batch of blocks before running its
// steps, so each batch waits on LDS once rather than once per block.

#include "common.h"

namespace nnh {
namespace {

constexpr int BF16_NT = 128;                // threads per workgroup
constexpr int BF16_D = 8;                   // 16-byte weight pieces in flight per lane
constexpr int BF16_X_LDS = 72 * 1024;       // LDS for staged x (all vectors of a pass)

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

// Steps of the chain paths: S = cols / C, in blocks of 8 (the last partial).
struct Bf16Geom {
    int C, S, nb8, XS;
    __host__ __device__ Bf16Geom(int c, int cols) : C(c), S(cols / c), nb8((cols / c + 7) / 8), XS(0) {
        XS = nb8 * 8 + 4;  // float stride of a chain's x row: 16-byte units at an odd stride
    }
};

// The chain layout: rows in groups of RW = 64 / C (the rows one wave runs),
// each group stored block by block, so that one wave's load of a block is
// 1 KB of consecutive bytes:
//   bl[r / RW][b][r % RW][c][0..8) = W[r][(8b + s) C + c]
// (0 past the row, and for the pad rows up to a whole group).
constexpr int BF16_BLOCK_ELEMS = 64 * 8;  // one block of one row group: RW * C lanes x 8 values

inline __host__ __device__ int bf16_groups(int rows, int C) { return (rows + 64 / C - 1) / (64 / C); }

// One thread per 16-byte piece.
__global__ void relayout_bf16_kernel(const uint16_t* __restrict__ raw, uint16_t* __restrict__ bl, int rows, int cols,
                                     int C) {
    const Bf16Geom g(C, cols);
    const int RW = 64 / C;
    const size_t p = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= (size_t)bf16_groups(rows, C) * g.nb8 * 64) return;
    const size_t gb = p / 64;  // group * nb8 + block
    const int lane = (int)(p % 64), b = (int)(gb % g.nb8), rr = lane / C, c = lane % C;
    const size_t r = gb / g.nb8 * RW + rr;
    uint32_t v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int s0 = 8 * b + 2 * k, s1 = s0 + 1;
        const uint32_t lo = r < (size_t)rows && s0 < g.S ? raw[r * cols + (size_t)s0 * C + c] : 0u;
        const uint32_t hi = r < (size_t)rows && s1 < g.S ? raw[r * cols + (size_t)s1 * C + c] : 0u;
        v[k] = lo | (hi << 16);
    }
    *(uint4*)(bl + p * 8) = make_uint4(v[0], v[1], v[2], v[3]);
}

// One block of 8 steps of a chain for `nt` vectors: x from LDS (XG false:
// xt[t][c][8b..8b+8), two 16-byte reads) or from global memory (XG true).
template <int T, bool XG, bool FULL>
__device__ __forceinline__ void bf16_block(float (&acc)[T], const uint4& wv, int b, int steps, int c, int nt,
                                           const float* xl, int XS, const float* __restrict__ x, size_t x_stride,
                                           int C) {
    const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int t = 0; t < T; ++t) {
        if (t >= nt) break;
        float xv[8];
        if (!XG) {
            const float* xp = xl + ((size_t)t * C + c) * XS + 8 * b;
            const float4 x0 = *(const float4*)xp, x1 = *(const float4*)(xp + 4);
            xv[0] = x0.x, xv[1] = x0.y, xv[2] = x0.z, xv[3] = x0.w;
            xv[4] = x1.x, xv[5] = x1.y, xv[6] = x1.z, xv[7] = x1.w;
        } else {
#pragma unroll
            for (int s = 0; s < 8; ++s)
                xv[s] = (FULL || s < steps) ? x[(size_t)t * x_stride + (size_t)(8 * b + s) * C + c] : 0.0f;
        }
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            if (FULL || s < steps) {
                const float w = (s & 1) ? bf16_hi(wd[s >> 1]) : bf16_lo(wd[s >> 1]);
                acc[t] = __builtin_fmaf(w, xv[s], acc[t]);
            }
        }
    }
}

// TREE 0: the hadd tree (4-row kernel); 1: hsum8 over 8 chains; 2: add8
// over 32 chains, then hsum8.
template <int TREE>
__device__ __forceinline__ float bf16_reduce(float a) {
    if (TREE == 0) {
        a = __fadd_rn(a, xor_get(a, 1));
        a = __fadd_rn(a, xor_get(a, 2));
        return __fadd_rn(a, xor_get(a, 4));
    }
    if (TREE == 2) {
        a = __fadd_rn(a, xor_get(a, 8));
        a = __fadd_rn(a, xor_get(a, 16));
    }
    a = __fadd_rn(a, xor_get(a, 4));
    a = __fadd_rn(a, xor_get(a, 1));
    return __fadd_rn(a, xor_get(a, 2));
}

typedef float bf16_f4u __attribute__((ext_vector_type(4), aligned(4)));

// xt[t][c][i] = x_t[i C + c] for the nt vectors (C = 8 or 32, so cols % 4 == 0
// and a 16-byte piece of x holds 4 consecutive columns); 8 pieces in flight
// per thread.
template <int NT>
__device__ __forceinline__ void stage_x(float* xl, const float* __restrict__ x, size_t x_stride, int nt, int cols,
                                        const Bf16Geom& g) {
    const int n4 = cols / 4;
    for (int t = 0; t < nt; ++t) {
        const float* xt = x + (size_t)t * x_stride;
        for (int p0 = threadIdx.x; p0 < n4; p0 += 8 * NT) {
            float4 v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                v[k] = __builtin_bit_cast(float4, *(const bf16_f4u*)(xt + 4 * min(p0 + k * NT, n4 - 1)));
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int p = p0 + k * NT;
                if (p < n4) {
                    const float e4[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int e = 4 * p + q, i = e / g.C, cc = e - i * g.C;
                        xl[((size_t)t * g.C + cc) * g.XS + i] = e4[q];
                    }
                }
            }
        }
    }
    __syncthreads();
}

// D 16-byte weight pieces of a lane, blocks b0 .. b0 + D (clamped to the last
// block: the extra loads are in bounds and their values unused).
template <int D>
__device__ __forceinline__ void load_pieces(uint4 (&wv)[D], const uint16_t* wp, int b0, int nb8) {
#pragma unroll
    for (int d = 0; d < D; ++d) wv[d] = load_nt16u(wp + (size_t)min(b0 + d, nb8 - 1) * BF16_BLOCK_ELEMS);
}

// D blocks of the chains for the T vectors. A batch of whole blocks with x in
// LDS reads each vector's 8 D x values first and then runs its 8 D steps, so
// the LDS latency is paid once per vector and batch; the vectors' chains are
// independent, the steps of each stay in order.
template <int C, int T, bool XG, int D>
__device__ __forceinline__ void run_pieces(float (&acc)[T], const uint4 (&wv)[D], int b0, int c, const float* xl,
                                           const Bf16Geom& g, const float* __restrict__ x, size_t x_stride) {
    const int full = g.S / 8;  // whole blocks; a partial one follows when S % 8 != 0
    if (!XG && b0 + D <= full) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float* xp = xl + ((size_t)t * C + c) * g.XS + 8 * b0;
            float4 xr[D][2];
#pragma unroll
            for (int d = 0; d < D; ++d) {
                xr[d][0] = *(const float4*)(xp + 8 * d);
                xr[d][1] = *(const float4*)(xp + 8 * d + 4);
            }
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const float xs[8] = {xr[d][0].x, xr[d][0].y, xr[d][0].z, xr[d][0].w,
                                     xr[d][1].x, xr[d][1].y, xr[d][1].z, xr[d][1].w};
                const uint32_t wd[4] = {wv[d].x, wv[d].y, wv[d].z, wv[d].w};
#pragma unroll
                for (int s = 0; s < 8; ++s)
                    acc[t] = __builtin_fmaf((s & 1) ? bf16_hi(wd[s >> 1]) : bf16_lo(wd[s >> 1]), xs[s], acc[t]);
            }
        }
        return;
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const int b = b0 + d;
        if (b < full)
            bf16_block<T, XG, true>(acc, wv[d], b, 8, c, T, xl, g.XS, x, x_stride, C);
        else if (b < g.nb8)
            bf16_block<T, XG, false>(acc, wv[d], b, g.S - 8 * b, c, T, xl, g.XS, x, x_stride, C);
    }
}

// C lanes per row (one chain each), NT / C rows per workgroup, T vectors per
// weight pass; D 16-byte weight pieces in flight per lane.
template <int C, int TREE, int T, bool XG, int D, int NT>
__global__ __launch_bounds__(NT) void gemv_bf16_kernel(const uint16_t* __restrict__ bl, int rows, int cols,
                                                       const float* __restrict__ x, size_t x_stride,
                                                       float* __restrict__ y, size_t y_stride) {
    extern __shared__ __align__(16) float xl[];
    const Bf16Geom g(C, cols);
    const int tid = threadIdx.x, c = tid % C;
    const int row_raw = blockIdx.x * (NT / C) + tid / C;
    // Loads stay inside the padded groups; the store is skipped past `rows`.
    const int row = min(row_raw, bf16_groups(rows, C) * (64 / C) - 1);
    const uint16_t* wp = bl + (size_t)(row / (64 / C)) * g.nb8 * BF16_BLOCK_ELEMS + (size_t)(row % (64 / C)) * C * 8 +
                         (size_t)c * 8;
    if (!XG) stage_x<NT>(xl, x, x_stride, T, cols, g);
    float acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = 0.0f;
    for (int b0 = 0; b0 < g.nb8; b0 += D) {
        uint4 wv[D];
        load_pieces<D>(wv, wp, b0, g.nb8);
        run_pieces<C, T, XG, D>(acc, wv, b0, c, xl, g, x, x_stride);
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const float v = bf16_reduce<TREE>(acc[t]);
        if (row_raw < rows && c == 0) y[(size_t)t * y_stride + row_raw] = v;
    }
}

// gemv_bf16_f64 (mod.rs:556-564): one thread per (vector, row).
__global__ void gemv_bf16_f64_kernel(const uint16_t* __restrict__ raw, int rows, int cols, const float* __restrict__ x,
                                     size_t x_stride, int n_tok, float* __restrict__ y, size_t y_stride) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)rows * n_tok) return;
    const size_t t = i / rows, r = i - t * rows;
    const uint16_t* w = raw + r * cols;
    const float* xt = x + t * x_stride;
    double s = 0.0;
    for (int k = 0; k < cols; ++k) s += (double)bf16f(w[k]) * (double)xt[k];
    y[t * y_stride + r] = (float)s;
}

// WeightFormat::Bf16's encoder (load.rs:198-202): f32_to_bf16 per element.
__global__ void encode_bf16_kernel(const float* __restrict__ w, size_t n, uint16_t* __restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = (uint16_t)f32_to_bf16(w[i]);
}

template <int C, int TREE, int T>
void launch_chain(const uint16_t* bl, int rows, int cols, const float* x, size_t x_stride, float* y, size_t y_stride,
                  bool xg, hipStream_t st) {
    const Bf16Geom g(C, cols);
    constexpr int D = BF16_D, NT = BF16_NT;
    const dim3 grid(ceil_div(rows, NT / C)), block(NT);
    if (xg)
        gemv_bf16_kernel<C, TREE, T, true, D, NT><<<grid, block, 0, st>>>(bl, rows, cols, x, x_stride, y, y_stride);
    else
        gemv_bf16_kernel<C, TREE, T, false, D, NT><<<grid, block, (size_t)T * C * g.XS * 4, st>>>(
            bl, rows, cols, x, x_stride, y, y_stride);
}

// Up to 4 vectors per weight pass, as many as the staged x of all of them fits
// BF16_X_LDS; each pass runs the kernel built for exactly its count.
template <int C, int TREE>
void launch_chains(const uint16_t* bl, int rows, int cols, const float* x, size_t x_stride, int n_tok, float* y,
                   size_t y_stride, hipStream_t st) {
    const Bf16Geom g(C, cols);
    const size_t per_tok = (size_t)C * g.XS * 4;
    const int tp = per_tok * 4 <= (size_t)BF16_X_LDS ? 4 : per_tok * 2 <= (size_t)BF16_X_LDS ? 2 : 1;
    const bool xg = per_tok > (size_t)BF16_X_LDS;  // too wide to stage: x from global memory
    for (int t0 = 0; t0 < n_tok; t0 += tp) {
        const int nt = n_tok - t0 < tp ? n_tok - t0 : tp;
        const float* xt = x + (size_t)t0 * x_stride;
        float* yt = y + (size_t)t0 * y_stride;
        switch (nt) {
            case 4: launch_chain<C, TREE, 4>(bl, rows, cols, xt, x_stride, yt, y_stride, xg, st); break;
            case 3: launch_chain<C, TREE, 3>(bl, rows, cols, xt, x_stride, yt, y_stride, xg, st); break;
            case 2: launch_chain<C, TREE, 2>(bl, rows, cols, xt, x_stride, yt, y_stride, xg, st); break;
            default: launch_chain<C, TREE, 1>(bl, rows, cols, xt, x_stride, yt, y_stride, xg, st); break;
        }
    }
}

}  // namespace

int bf16_path(size_t rows, size_t cols) {
    if (cols % 8 != 0) return BF16_PATH_F64;
    if (rows % 4 == 0) return BF16_PATH_QUAD;
    return cols % 32 == 0 ? BF16_PATH_ROW32 : BF16_PATH_ROW8;
}

size_t bf16_layout_bytes(int path, size_t rows, size_t cols) {
    if (path == BF16_PATH_F64) return 0;
    const Bf16Geom g(path == BF16_PATH_ROW32 ? 32 : 8, (int)cols);
    return (size_t)bf16_groups((int)rows, g.C) * g.nb8 * BF16_BLOCK_ELEMS * 2;
}

void launch_relayout_bf16(int path, const uint16_t* raw, uint16_t* bl, int rows, int cols, hipStream_t st) {
    if (path == BF16_PATH_F64) return;
    const int C = path == BF16_PATH_ROW32 ? 32 : 8;
    const Bf16Geom g(C, cols);
    const size_t pieces = (size_t)bf16_groups(rows, C) * g.nb8 * 64;
    relayout_bf16_kernel<<<(unsigned)((pieces + 255) / 256), 256, 0, st>>>(raw, bl, rows, cols, C);
}

void launch_gemv_bf16(int path, const uint16_t* raw, const uint16_t* bl, int rows, int cols, const float* x,
                      size_t x_stride, int n_tok, float* y, size_t y_stride, hipStream_t st) {
    if (path == BF16_PATH_F64) {
        const size_t n = (size_t)rows * n_tok;
        gemv_bf16_f64_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(raw, rows, cols, x, x_stride, n_tok, y,
                                                                           y_stride);
    } else if (path == BF16_PATH_QUAD) {
        launch_chains<8, 0>(bl, rows, cols, x, x_stride, n_tok, y, y_stride, st);
    } else if (path == BF16_PATH_ROW8) {
        launch_chains<8, 1>(bl, rows, cols, x, x_stride, n_tok, y, y_stride, st);
    } else {
        launch_chains<32, 2>(bl, rows, cols, x, x_stride, n_tok, y, y_stride, st);
    }
}

void launch_encode_bf16(const float* w, size_t n, uint16_t* out, hipStream_t st) {
    encode_bf16_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(w, n, out);
}

}  // namespace nnh
