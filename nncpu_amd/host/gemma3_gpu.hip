// The Gemma-3 decode step resident on the GPU: the forward of gemma3.cpp
// (crates/nncpu/src/model/forward.rs:197-439, 719-965 with the scalar.rs
// non-matmul kernels) for one token, with every operation in the same order
// and rounding as that CPU restatement, so a decode gives the same tokens and
// the same per-layer hidden states bit for bit. The token and the position
// live in device memory, and one step is captured once in a HIP graph and
// replayed per generated token: no host round trip inside the decode loop.
//
// Five kernels per layer. Every kernel boundary costs a few microseconds on
// this GPU, so the non-matmul work rides on the matmul kernels around it:
//   qkv   the previous layer's post-FFW RMSNorm and residual add (or, in
//         layer 0, the embedding row), the attention RMSNorm, then the q, k
//         and v matmuls (one launch over the three matrices);
//   attn  the q / k RMSNorms, NeoX RoPE, the K/V append and the attention,
//         one workgroup per query head;
//   o     the output projection (the library's one-vector kernel);
//   ffn   the post-attention RMSNorm and residual, the FFN RMSNorm, then the
//         gate and up matmuls with GELU(gate) * up in the epilogue (a
//         workgroup runs eight rows of each);
//   down  the down projection (the library's one-vector kernel).
// The residual and norm prologue is recomputed by every workgroup of its
// kernel (the same operations, so the same bits), while the weight loads of
// the matmul are already in flight; workgroup 0 stores the new residual.
// The residual stream alternates between two buffers, so no kernel reads the
// buffer it writes. The matmuls are the library's bit-exact f32 path: its
// one-vector core (f32_m1.h) on the 16-lane weight layout that
// nnh_weight_f32_layout exposes, and nnh_model_argmax_dev for the lm_head
// (its first argmax stage fused into the gemv).
//
// What is taken from the host: RoPE's cos / sin per position (computed with
// the CPU restatement's own libm calls, uploaded once) and the embedding
// scale sqrt(n_embd). The attention runs in one key block (n_ctx <= 256, the
// reference's ATTN_BLOCK), so the block merge, whose exp is libm's, never
// runs; longer contexts are refused. Compiled with -ffp-contract=off;
// __fmaf_rn / __fma_rn exactly where the CPU code calls std::fma.

#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "f32_m1.h"
#include "gemma3.h"
#include "nncpu_hip.h"

namespace {

using nnh::F32Mat;
using nnh::lds_barrier;
using nnh::ScaleStage;
using nnh::M1Lane;
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef float f4u __attribute__((ext_vector_type(4), aligned(4)));

constexpr int ATTN_BLOCK = 256;  // model/mod.rs:84-87
constexpr int WG = 256;          // threads per workgroup
constexpr int E_MAX = 2048;      // residual width

__device__ __forceinline__ float bf16f(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ uint16_t to_bf16(float f) {
    const uint32_t u = __float_as_uint(f);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
// hsum8 of lanes 0..7's values, by lane exchanges (valid at lane 0):
// xor-4 gives v_l + v_{l+4}, xor-1 and xor-2 then add those pairs as hsum8 does.
__device__ __forceinline__ float hsum8_lanes(float a) {
    const float p = __fadd_rn(a, __shfl_xor(a, 4, 64));
    const float q = __fadd_rn(p, __shfl_xor(p, 1, 64));
    return __fadd_rn(q, __shfl_xor(q, 2, 64));
}
__device__ __forceinline__ float4 ld4(const float* p) { return __builtin_bit_cast(float4, *(const f4u*)p); }

// scalar.rs:19-84 (gemma3.cpp exp_lane).
__device__ float exp_lane(float x) {
    const float EXP_LO = -87.336544f, EXP_HI = 88.722839f;
    const float LOG2E = 1.44269504088896340736f, LN2_HI = 0.693359375f, LN2_LO = -2.12194440e-4f;
    x = x > EXP_LO ? x : EXP_LO;
    x = x < EXP_HI ? x : EXP_HI;
    const float fx = __fsub_rn(__fadd_rn(__fmul_rn(x, LOG2E), 12582912.0f), 12582912.0f);
    float r = __fmaf_rn(-fx, LN2_HI, x);
    r = __fmaf_rn(-fx, LN2_LO, r);
    float y = __fmaf_rn(1.9875691500e-4f, r, 1.3981999507e-3f);
    y = __fmaf_rn(y, r, 8.3334519073e-3f);
    y = __fmaf_rn(y, r, 4.1665795894e-2f);
    y = __fmaf_rn(y, r, 1.6666665459e-1f);
    y = __fmaf_rn(y, r, 5.0000001201e-1f);
    y = __fmaf_rn(y, __fmul_rn(r, r), r);
    y = __fadd_rn(y, 1.0f);
    const float p2 = __uint_as_float((uint32_t)((int32_t)fx + 127) << 23);
    return __fmul_rn(y, p2);
}

// scalar.rs:86-103 (gemma3.cpp gelu_lane).
__device__ float gelu_lane(float v) {
    const float GELU_C = 0.79788456080286535f, GELU_A = 0.044715f;
    const float v3 = __fmul_rn(__fmul_rn(v, v), v);
    const float u = __fmul_rn(GELU_C, __fmaf_rn(GELU_A, v3, v));
    const float u2 = __fmul_rn(u, u), u4 = __fmul_rn(u2, u2), u6 = __fmul_rn(u4, u2);
    const float num = __fmul_rn(u, __fadd_rn(u6, __fmaf_rn(378.0f, u4, __fmaf_rn(17325.0f, u2, 135135.0f))));
    const float den = __fmaf_rn(28.0f, u6, __fmaf_rn(3150.0f, u4, __fmaf_rn(62370.0f, u2, 135135.0f)));
    const float t = fabsf(u) >= 5.0f ? copysignf(1.0f, u) : __fdiv_rn(num, den);
    return __fmul_rn(__fmul_rn(0.5f, v), __fadd_rn(1.0f, t));
}

// A chain input in LDS, transposed: element e of a dim-vector (dim a
// multiple of 128) at (e % 8) * S + e / 8, S = dim / 8 + 4, so FMA lane l's
// values are contiguous (16-byte reads) and the 4-float pad spreads the eight
// lanes' reads over the banks.
__device__ __forceinline__ int tstride(int dim) { return dim / 8 + 4; }
__device__ __forceinline__ void tput4(float* xt, int S, int piece, float4 v) {
    float* p = xt + 4 * (piece & 1) * S + (piece >> 1);
    p[0] = v.x;
    p[S] = v.y;
    p[2 * S] = v.z;
    p[3 * S] = v.w;
}

// hsum8 of the eight FMA lanes' sums of squares of a transposed dim-vector
// (dim % 128 == 0), run by lanes 0..7 of the calling wave; valid at lane 0.
// A lane's values are read from LDS 12 float4s at a time, all issued before
// that chunk's FMAs (a buffer rotated across loop iterations instead makes
// the compiler wait for every read at the loop head).
__device__ __forceinline__ float chain_sumsq(const float* xt, int dim, int lane) {
    constexpr int CH = 12;
    float a = 0.0f;
    if (lane < 8) {
        const float4* p = (const float4*)(xt + lane * tstride(dim));
        const int n = dim / 32;
        for (int m = 0; m < n; m += CH) {
            float4 b[CH];
#pragma unroll
            for (int k = 0; k < CH; ++k) b[k] = p[min(m + k, n - 1)];  // past the end: a spare read
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                if (m + k < n) {
                    a = __fmaf_rn(b[k].x, b[k].x, a);
                    a = __fmaf_rn(b[k].y, b[k].y, a);
                    a = __fmaf_rn(b[k].z, b[k].z, a);
                    a = __fmaf_rn(b[k].w, b[k].w, a);
                }
            }
        }
    }
    return hsum8_lanes(a);
}

// The RMSNorm scale of a transposed dim-vector xt (scalar.rs:232-292,
// gemma3.cpp sum_sq / rmsnorm_gamma_multi): lanes 0..7 of wave 0 run the
// eight FMA lanes over the chunks of 8 in order, hsum8, lane 0 forms
// (float)(1 / sqrt(ss * inv_dim + eps)) in f64 (dim % 8 == 0: no tail).
// xt written before a barrier; every thread gets the scale (bc: one LDS float).
__device__ float wg_rms_scale(const float* xt, int dim, float eps, float* bc) {
    const int tid = threadIdx.x;
    if (tid < 64) {
        const float r = chain_sumsq(xt, dim, tid);
        if (tid == 0) {
            const float inv_dim = __fdiv_rn(1.0f, (float)dim);
            bc[0] = (float)__ddiv_rn(1.0, __dsqrt_rn(__dadd_rn(__dmul_rn((double)r, (double)inv_dim), (double)eps)));
        }
    }
    lds_barrier();
    return bc[0];
}

// ---- the matmul kernels' prologues --------------------------------------------------------
// NT threads per workgroup; a thread holds pieces (4 floats) tid + NT k of
// an E-vector.

template <int NT>
struct Pieces {
    static constexpr int K = (E_MAX / 4 + NT - 1) / NT;
};

// A prologue's inputs: the block output o, the residual x, two gammas.
template <int NT>
struct ResIn {
    static constexpr int K = Pieces<NT>::K;
    float4 o[K], x[K], g1[K], g2[K];
    __device__ __forceinline__ void load(const float* po, const float* px, const float* pg1, const float* pg2, int E) {
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int i = 4 * min((int)threadIdx.x + NT * k, E / 4 - 1);
            o[k] = ld4(po + i);
            x[k] = ld4(px + i);
            g1[k] = ld4(pg1 + i);
            g2[k] = ld4(pg2 + i);
        }
    }
};

__device__ __forceinline__ float4 add_normed(float4 x, float4 o, float s, float4 g) {
    return make_float4(__fadd_rn(x.x, __fmul_rn(__fmul_rn(o.x, s), g.x)),
                       __fadd_rn(x.y, __fmul_rn(__fmul_rn(o.y, s), g.y)),
                       __fadd_rn(x.z, __fmul_rn(__fmul_rn(o.z, s), g.z)),
                       __fadd_rn(x.w, __fmul_rn(__fmul_rn(o.w, s), g.w)));
}
__device__ __forceinline__ float4 normed(float4 x, float s, float4 g) {
    return make_float4(__fmul_rn(__fmul_rn(x.x, s), g.x), __fmul_rn(__fmul_rn(x.y, s), g.y),
                       __fmul_rn(__fmul_rn(x.z, s), g.z), __fmul_rn(__fmul_rn(x.w, s), g.w));
}

// Piece index of thread slot k, and whether it is one of the vector's own
// (slots past the end repeat the last piece: stores of it write its own
// values again, so they need no condition).
template <int NT>
__device__ __forceinline__ int piece(int k, int E) { return min((int)threadIdx.x + NT * k, E / 4 - 1); }

// y = RMSNorm(x, g) into LDS yl, x already in LDS xs (transposed) and in the
// thread's registers; ends with a barrier.
template <int NT, int K>
__device__ __forceinline__ void norm_to(const float4 (&xn)[K], const float4 (&g)[K], int E, float eps,
                                        const float* xs, float* yl, float* bc) {
    const float s = wg_rms_scale(xs, E, eps, bc);
#pragma unroll
    for (int k = 0; k < K; ++k) *(float4*)(yl + 4 * piece<NT>(k, E)) = normed(xn[k], s, g[k]);
    lds_barrier();
}

// Keep x (the new residual) in xs (transposed) and, from workgroup 0, in
// x_out and rec.
template <int NT, int K>
__device__ __forceinline__ void keep_residual(const float4 (&xn)[K], int E, float* xs, float* x_out, float* rec) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = piece<NT>(k, E);
        tput4(xs, tstride(E), i, xn[k]);
        if (blockIdx.x == 0) {
            *(float4*)(x_out + 4 * i) = xn[k];
            if (rec) *(float4*)(rec + 4 * i) = xn[k];
        }
    }
    lds_barrier();
}

// x_new = x + RMSNorm(o, g1), y = RMSNorm(x_new, g2) (forward.rs:749-803):
// a block's post-norm and residual add, then the next pre-norm. y goes to
// LDS yl (the matmul's x). xs: LDS scratch of E + 32 floats. In two parts:
// res_stage puts o in LDS (so every input load has landed when it returns),
// res_norm does the rest.
template <int NT>
__device__ __forceinline__ void res_stage(const ResIn<NT>& r, int E, float* xs) {
#pragma unroll
    for (int k = 0; k < Pieces<NT>::K; ++k) tput4(xs, tstride(E), piece<NT>(k, E), r.o[k]);
    lds_barrier();
}

template <int NT>
__device__ void res_norm(const ResIn<NT>& r, int E, float eps, float* xs, float* yl, float* bc, float* x_out,
                         float* rec) {
    constexpr int K = Pieces<NT>::K;
    const float s1 = wg_rms_scale(xs, E, eps, bc);
    float4 xn[K];
#pragma unroll
    for (int k = 0; k < K; ++k) xn[k] = add_normed(r.x[k], r.o[k], s1, r.g1[k]);
    keep_residual<NT>(xn, E, xs, x_out, rec);
    norm_to<NT>(xn, r.g2, E, eps, xs, yl, bc);
}

// Layer 0's input: the token's Q8_0 row of the tied token_embd times
// sqrt(n_embd) (kernels/mod.rs:917-929: f32(q) * (bf16(s) * scale)).
template <int NT>
struct EmbIn {
    static constexpr int K = Pieces<NT>::K;
    uint32_t q[K], s[K];  // four quants, their block's BF16 scale
    float4 g[K];
    __device__ __forceinline__ void load(const uint64_t* tok, const int8_t* tq, const uint16_t* ts, const float* pg,
                                         int E) {
        const size_t t = (size_t)*tok;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int i = 4 * piece<NT>(k, E);
            q[k] = *(const uint32_t*)(tq + t * E + i);
            s[k] = ts[t * (E / 32) + i / 32];
            g[k] = ld4(pg + i);
        }
    }
};

template <int NT>
__device__ void emb_norm(const EmbIn<NT>& r, int E, float eps, float embd_scale, float* xs, float* yl, float* bc,
                         float* x_out) {
    constexpr int K = Pieces<NT>::K;
    float4 xn[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const float vs = __fmul_rn(bf16f(r.s[k]), embd_scale);
        xn[k] = make_float4(__fmul_rn((float)(int8_t)(r.q[k] & 0xffu), vs), __fmul_rn((float)(int8_t)(r.q[k] >> 8), vs),
                            __fmul_rn((float)(int8_t)(r.q[k] >> 16), vs), __fmul_rn((float)(int8_t)(r.q[k] >> 24), vs));
    }
    keep_residual<NT>(xn, E, xs, x_out, nullptr);
    norm_to<NT>(xn, r.g, E, eps, xs, yl, bc);
}

// ---- the step's kernels -----------------------------------------------------------------
// One workgroup per CU for the matmul kernels (the grids stay under 256
// workgroups), so the wave that runs a norm's FMA chain has its SIMD to
// itself while the others wait at the barrier.

constexpr int QKV_NT = 512;   // 32 rows of one matrix per workgroup
constexpr int FFN_NT = 1024;  // 32 gate rows and the same 32 up rows
constexpr int MAX_NBP = E_MAX / 32;

struct QkvArgs {
    F32Mat m[3];  // q, k, v
    float* y[3];
    int wg[3];  // workgroups per matrix
    const float *o, *x_in, *post, *norm;  // post: the previous layer's post-FFW gamma; norm: attention's
    float* x_out;
    float* rec;  // this layer's slot of the step-0 record (advanced by *step_p * rec_stride), or null
    const int* step_p;
    size_t rec_stride;
    const uint64_t* tok;  // layer 0: the token and the embedding table
    const int8_t* tq;
    const uint16_t* ts;
    float embd_scale;
    int E;
    float eps;
};

template <int D, bool FIRST>
__global__ __launch_bounds__(QKV_NT) void qkv_kernel(QkvArgs a) {
    constexpr int NT = QKV_NT, R = NT / 16;
    __shared__ __attribute__((aligned(16))) float xs[E_MAX + 32];
    __shared__ __attribute__((aligned(16))) float yl[E_MAX];
    __shared__ __attribute__((aligned(16))) uint16_t sl[R * MAX_NBP];
    __shared__ float bc[4];
    const int tid = threadIdx.x;
    ResIn<NT> r;
    EmbIn<NT> e;
    if (FIRST)
        e.load(a.tok, a.tq, a.ts, a.norm, a.E);
    else
        r.load(a.o, a.x_in, a.post, a.norm, a.E);
    int b = blockIdx.x, seg = 0;
    if (b >= a.wg[0]) {
        b -= a.wg[0];
        seg = 1;
        if (b >= a.wg[1]) {
            b -= a.wg[1];
            seg = 2;
        }
    }
    const F32Mat m = a.m[seg];
    const int row0 = b * R, row_raw = row0 + (tid >> 4);
    const int row = row_raw < m.rows ? row_raw : m.rows - 1;  // keep loads in bounds; the store is skipped
    ScaleStage<NT, R * MAX_NBP * 2> ss;
    ss.load(m, row0, min(R, m.rows - row0));
    M1Lane<1, D> L;
    L.init(m, row, tid & 15);
    // The prologue's inputs land first; the weight loads then stream while
    // the prologue's norm chains run (issued earlier, they would queue
    // ahead of other workgroups' prologue loads).
    ss.store(sl);
    if (!FIRST) res_stage<NT>(r, a.E, xs);
    __builtin_amdgcn_s_waitcnt(NNH_VMCNT(0));  // every prologue load has landed
    __builtin_amdgcn_sched_barrier(0);
    L.prefetch();
    __builtin_amdgcn_sched_barrier(0);
    if (FIRST)
        emb_norm<NT>(e, a.E, a.eps, a.embd_scale, xs, yl, bc, a.x_out);
    else
        res_norm<NT>(r, a.E, a.eps, xs, yl, bc, a.x_out, a.rec ? a.rec + (size_t)*a.step_p * a.rec_stride : nullptr);
    L.run(yl, sl + (row - row0) * m.nbp);
    const float v = L.reduce();
    if (row_raw < m.rows && (tid & 15) == 0) a.y[seg][row_raw] = v;
}

struct FfnArgs {
    F32Mat gate, up;
    float* h;  // GELU(gate) * up
    int F;
    const float *o, *x_in, *post, *norm;  // post_attention_norm, ffn_norm
    float* x_out;
    int E;
    float eps;
};

// Workgroup g runs gate rows 32g..32g+31 (row slots 0..31) and the same up
// rows (slots 32..63); h = GELU(gate) * up (forward.rs:771-777).
template <int D>
__global__ __launch_bounds__(FFN_NT) void ffn_kernel(FfnArgs a) {
    constexpr int NT = FFN_NT, R = NT / 16, HR = R / 2;
    __shared__ __attribute__((aligned(16))) float xs[E_MAX + 32];
    __shared__ __attribute__((aligned(16))) float yl[E_MAX];
    __shared__ __attribute__((aligned(16))) uint16_t sl[R * MAX_NBP];
    __shared__ float bc[4], res[R];
    const int tid = threadIdx.x, slot = tid >> 4, r0 = blockIdx.x * HR;
    ResIn<NT> r;
    r.load(a.o, a.x_in, a.post, a.norm, a.E);
    const int nr = min(HR, a.F - r0);
    ScaleStage<NT, HR * MAX_NBP * 2> sg, su;
    sg.load(a.gate, r0, nr);
    su.load(a.up, r0, nr);
    const int row = r0 + (slot % HR) < a.F ? r0 + (slot % HR) : a.F - 1;
    M1Lane<1, D> L;
    L.init(slot < HR ? a.gate : a.up, row, tid & 15);
    // The prologue's inputs land first; the weight loads then stream while
    // the norm chains run.
    sg.store(sl);
    su.store(sl + HR * a.gate.nbp);
    res_stage<NT>(r, a.E, xs);
    __builtin_amdgcn_s_waitcnt(NNH_VMCNT(0));  // every prologue load has landed
    __builtin_amdgcn_sched_barrier(0);
    L.prefetch();
    __builtin_amdgcn_sched_barrier(0);
    res_norm<NT>(r, a.E, a.eps, xs, yl, bc, a.x_out, nullptr);
    L.run(yl, sl + (slot < HR ? row - r0 : HR + row - r0) * a.gate.nbp);
    const float v = L.reduce();
    if ((tid & 15) == 0) res[slot] = v;
    lds_barrier();
    if (tid < HR && r0 + tid < a.F) a.h[r0 + tid] = __fmul_rn(gelu_lane(res[tid]), res[HR + tid]);
}

struct FinalArgs {
    const float *o, *x_in, *post, *norm;  // the last post-FFW gamma, output_norm
    float *x_out, *y, *rec;
    const int* step_p;
    size_t rec_stride;
    int E;
    float eps;
};

// After the last layer: its residual, then y = RMSNorm(x, output_norm).
__global__ __launch_bounds__(WG) void final_kernel(FinalArgs a) {
    __shared__ __attribute__((aligned(16))) float xs[E_MAX + 32];
    __shared__ __attribute__((aligned(16))) float yl[E_MAX];
    __shared__ float bc[4];
    ResIn<WG> r;
    r.load(a.o, a.x_in, a.post, a.norm, a.E);
    res_stage<WG>(r, a.E, xs);
    res_norm<WG>(r, a.E, a.eps, xs, yl, bc, a.x_out, a.rec + (size_t)*a.step_p * a.rec_stride);
    for (int i = threadIdx.x; i < a.E / 4; i += WG) *(float4*)(a.y + 4 * i) = *(const float4*)(yl + 4 * i);
}

struct AttnArgs {
    const float *q, *k, *v;  // the projections
    const float *q_norm, *k_norm, *cos_t, *sin_t;
    const int* pos_p;
    uint16_t *kc, *vc;  // this layer's caches [n_ctx][n_kv * HD]
    int group, KV, window;
    float scale, eps;
    float* out;
};

// The first-maximum scan's step (scalar.rs attn_block): b follows a.
__device__ __forceinline__ float first_max(float a, float b) { return a < b ? b : a; }

// Attention workgroups per query head: each runs every score of its head
// and the V chains of HD / ATTN_SPLIT output elements.
constexpr int ATTN_SPLIT = 8;
// Threads per attention workgroup: all 16 waves issue the cache loads (a
// wave keeps only a few loads in flight), the first 4 do the rest.
constexpr int ATTN_NT = 1024;

// One query head, one key block (forward.rs:326-351 and attn_block /
// attn_finish, scalar.rs:444-548): q / k RMSNorm, NeoX RoPE at the current
// position, the K/V append (by one workgroup per KV head), scores by 8-lane
// FMA dots and hsum8 times the scale, the first maximum, exp_lane, the
// 8-lane sum of the weights over whole chunks then the tail in order, and
// the V sum as one FMA chain per output element over the keys in order,
// / sum. Workgroup (h, e) of ATTN_SPLIT per head computes all of head h's
// scores (thread t scores key t) and output elements e * EW .. e * EW + EW - 1.
// The cached keys 0..n-2 and the workgroup's slice of their values are
// copied into LDS at the start by coalesced direct loads; a key row's
// 16-byte chunks are stored XOR-swizzled by the row index, so the score
// threads (one row each) read different banks. The new key and value come
// from LDS.
template <int HD>
__global__ __launch_bounds__(ATTN_NT) void attn_kernel(AttnArgs a) {
    static_assert(HD % 64 == 0 && HD <= WG && ATTN_BLOCK <= WG, "head size, key block");
    constexpr int HALF = HD / 2, CH = HD / 8, EW = HD / ATTN_SPLIT, VCH = EW / 8;
    constexpr int ST = ATTN_BLOCK / 8 + 4;  // transposed weights: lane l's run at l * ST
    constexpr int VS = ATTN_BLOCK + 8;  // transposed value rows: element e's keys at e * VS
    constexpr int VL = (ATTN_BLOCK * VCH + ATTN_NT - 1) / ATTN_NT;  // value pieces per thread
    constexpr int QS = CH + 4;  // qe row stride: 16-byte rows, the pad spreads the four lanes' reads
    __shared__ __attribute__((aligned(16))) uint16_t ks_lds[ATTN_BLOCK * HD];
    __shared__ __attribute__((aligned(16))) uint16_t vt[EW * VS];
    __shared__ __attribute__((aligned(16))) float qs[HD];
    __shared__ __attribute__((aligned(16))) float ks[HD];
    __shared__ __attribute__((aligned(16))) float qt[HD + 32];
    __shared__ __attribute__((aligned(16))) float qe[8 * QS];  // rotated q by element of chunk: qe[e * QS + c] = q[8c + e]
    __shared__ __attribute__((aligned(16))) float kt[HD + 32];
    __shared__ __attribute__((aligned(16))) uint16_t kn[HD];
    __shared__ __attribute__((aligned(16))) float sc[ATTN_BLOCK];
    __shared__ __attribute__((aligned(16))) float sct[8 * ST];
    __shared__ float red[2 + ATTN_NT / 64 + 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pos = *a.pos_p, h = blockIdx.x / ATTN_SPLIT, es = blockIdx.x % ATTN_SPLIT, kvh = h / a.group;
    const int first = (a.window > 0 && pos + 1 > a.window) ? pos + 1 - a.window : 0;
    const int n = pos + 1 - first;  // keys; the last is the new one
    const size_t kv_dim = (size_t)a.KV * HD;
    const int i = tid < HD ? tid : HD - 1;
    const float qv = a.q[h * HD + i], kv = a.k[kvh * HD + i];
    const float vv = a.v[kvh * HD + es * EW + (tid < EW ? tid : EW - 1)];
    const float qg = a.q_norm[i], kg = a.k_norm[i];
    const float cs = a.cos_t[(size_t)pos * HALF + i % HALF], sn = a.sin_t[(size_t)pos * HALF + i % HALF];
    // This slice of the cached values (keys first .. pos - 1), 16-byte pieces
    // into registers (a fixed count per thread, clamped), stored transposed
    // into LDS once they land.
    const uint16_t* vbase = a.vc + kvh * HD + es * EW + (size_t)first * kv_dim;
    const int nv = max((n - 1) * VCH, 1);
    uint4 vr[VL];
#pragma unroll
    for (int k = 0; k < VL; ++k) {
        const int u = min(tid + ATTN_NT * k, nv - 1);
        vr[k] = *(const uint4*)(vbase + (size_t)(u / VCH) * kv_dim + 8 * (u % VCH));
    }
    // Cached keys, 16 bytes per lane straight into LDS, 1 KB per wave
    // instruction; pieces past the end repeat the last one (their LDS slots
    // are never read).
    {
        const uint16_t* kbase = a.kc + kvh * HD + (size_t)first * kv_dim;
        const int nk = (n - 1) * CH, nik = (nk + 63) / 64;
        for (int k = wave; k < nik; k += ATTN_NT / 64) {
            const int u = min(64 * k + lane, nk - 1);
            const int t = u / CH, c = u % CH;  // LDS chunk c of row t holds key chunk c ^ (t % CH)
            __builtin_amdgcn_global_load_lds((const void*)(kbase + (size_t)t * kv_dim + 8 * (c ^ (t % CH))),
                                             (lds_ptr_t)(ks_lds + 512 * k), 16, 0, 0);
        }
    }
    // q and k RMSNorm: wave 0 runs q's chains, wave 1 k's (transposed copies).
    if (tid < HD) {
        qt[(tid & 7) * tstride(HD) + (tid >> 3)] = qv;
        kt[(tid & 7) * tstride(HD) + (tid >> 3)] = kv;
    }
    lds_barrier();
    if (wave < 2) {
        const float ss = chain_sumsq(wave == 0 ? qt : kt, HD, lane);
        if (lane == 0) {
            const float inv_dim = __fdiv_rn(1.0f, (float)HD);
            red[wave] = (float)__ddiv_rn(1.0, __dsqrt_rn(__dadd_rn(__dmul_rn((double)ss, (double)inv_dim), (double)a.eps)));
        }
    }
    lds_barrier();
    if (tid < HD) {
        qs[tid] = __fmul_rn(__fmul_rn(qv, red[0]), qg);
        ks[tid] = __fmul_rn(__fmul_rn(kv, red[1]), kg);
    }
    if (tid < EW) vt[tid * VS + n - 1] = to_bf16(vv);  // the new value: key n - 1
    lds_barrier();
    // RoPE: threads 0..HALF-1 rotate q's pairs (j, j + HALF), HALF..HD-1 k's.
    if (tid < HALF) {
        const float x0 = qs[tid], x1 = qs[tid + HALF];
        const float r0 = __fsub_rn(__fmul_rn(cs, x0), __fmul_rn(sn, x1));
        const float r1 = __fadd_rn(__fmul_rn(sn, x0), __fmul_rn(cs, x1));
        qe[(tid & 7) * QS + (tid >> 3)] = r0;
        qe[((tid + HALF) & 7) * QS + ((tid + HALF) >> 3)] = r1;
    } else if (tid < HD) {
        const int j = tid - HALF;
        const float x0 = ks[j], x1 = ks[j + HALF];
        kn[j] = to_bf16(__fsub_rn(__fmul_rn(cs, x0), __fmul_rn(sn, x1)));
        kn[j + HALF] = to_bf16(__fadd_rn(__fmul_rn(sn, x0), __fmul_rn(cs, x1)));
    }
    // The cached keys and values have landed (each wave its own copies,
    // then the barrier for the others').
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int k = 0; k < VL; ++k) {
        const int u = tid + ATTN_NT * k;
        if (u < (n - 1) * VCH) {
            const int t = u / VCH, e0 = 8 * (u % VCH);
            const uint32_t w[4] = {vr[k].x, vr[k].y, vr[k].z, vr[k].w};
#pragma unroll
            for (int q = 0; q < 8; ++q) vt[(e0 + q) * VS + t] = (uint16_t)(w[q / 2] >> (16 * (q & 1)));
        }
    }
    lds_barrier();
    if (h % a.group == 0 && tid < HD) {
        if (es == 0) a.kc[(size_t)pos * kv_dim + kvh * HD + tid] = kn[tid];
        if (tid < EW) a.vc[(size_t)pos * kv_dim + kvh * HD + es * EW + tid] = vt[tid * VS + n - 1];
    }
    // Scores: four lanes per key (key tid / 4), lane u running the dot's
    // chains u and u + 4 (elements 8c + u and 8c + u + 4, c in order), then
    // (a_u + a_{u+4}), xor-1, xor-2: hsum8's additions in its order. Each
    // lane's q values are contiguous in qe; a key chunk's two values are two
    // 32-bit LDS reads.
    {
        const int t = tid >> 2, u = tid & 3;
        float a0 = 0.0f, a1 = 0.0f;
        if (t < n) {
            const bool last = t == n - 1;
            const uint16_t* krow = last ? kn : ks_lds + t * HD;
            const int sw = last ? 0 : t % CH;
            const float* q0 = qe + u * QS;
            const float* q1 = qe + (u + 4) * QS;
            const int hs = 16 * (u & 1);
#pragma unroll
            for (int c0 = 0; c0 < CH; c0 += 4) {
                const float4 qa = *(const float4*)(q0 + c0), qb = *(const float4*)(q1 + c0);
                const float qav[4] = {qa.x, qa.y, qa.z, qa.w}, qbv[4] = {qb.x, qb.y, qb.z, qb.w};
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) {
                    const uint32_t* kc = (const uint32_t*)(krow + 8 * ((c0 + cc) ^ sw));
                    const uint32_t klo = kc[u >> 1], khi = kc[2 + (u >> 1)];
                    a0 = __fmaf_rn(qav[cc], bf16f((klo >> hs) & 0xffffu), a0);
                    a1 = __fmaf_rn(qbv[cc], bf16f((khi >> hs) & 0xffffu), a1);
                }
            }
        }
        float p = __fadd_rn(a0, a1);
        p = __fadd_rn(p, __shfl_xor(p, 1, 64));
        p = __fadd_rn(p, __shfl_xor(p, 2, 64));
        if (t < n && u == 0) sc[t] = __fmul_rn(p, a.scale);
    }
    lds_barrier();
    const float s_t = tid < n ? sc[tid] : -INFINITY;
    // The first maximum over keys in order: a leftmost-maximum tree, with a
    // NaN after key 0 never taken (as the scan's comparison never takes one)
    // and a NaN at key 0 kept (it is never replaced).
    float mv = (tid > 0 && s_t != s_t) ? -INFINITY : s_t;
#pragma unroll
    for (int k = 1; k < 64; k <<= 1) {
        const float o = __shfl_xor(mv, k, 64);
        mv = (lane & k) ? first_max(o, mv) : first_max(mv, o);
    }
    if (lane == 0) red[2 + wave] = mv;
    lds_barrier();
    float m = red[2];
#pragma unroll
    for (int w = 1; w < ATTN_NT / 64; ++w) m = first_max(m, red[2 + w]);
    if (tid < n) {
        const float pw = exp_lane(__fsub_rn(s_t, m));
        sc[tid] = pw;
        sct[(tid & 7) * ST + (tid >> 3)] = pw;
    }
    lds_barrier();
    if (tid < 64) {
        // The eight add lanes over the whole chunks of 8, in order.
        const int body = n & ~7, K = body / 8;
        float acc = 0.0f;
        if (tid < 8) {
            const float* p = sct + tid * ST;
            int k = 0;
            for (; k + 4 <= K; k += 4) {
                const float4 v = *(const float4*)(p + k);
                acc = __fadd_rn(__fadd_rn(__fadd_rn(__fadd_rn(acc, v.x), v.y), v.z), v.w);
            }
            for (; k < K; ++k) acc = __fadd_rn(acc, p[k]);
        }
        float l = hsum8_lanes(acc);
        if (tid == 0) {
            for (int j = body; j < n; ++j) l = __fadd_rn(l, sc[j]);
            red[2 + ATTN_NT / 64] = l > 0.0f ? __fdiv_rn(1.0f, l) : 0.0f;
        }
    }
    lds_barrier();
    if (tid < EW) {
        // V: one FMA chain per element over the keys in order, 8 keys per
        // 16-byte read of the transposed values (and two of the weights),
        // the next batch's reads issued before this batch's FMAs.
        const uint16_t* vrow = vt + tid * VS;
        const int nbat = (n + 7) / 8;
        float o = 0.0f;
        uint4 va, vb;
        float4 pa0, pa1, pb0, pb1;
        auto fetch = [&](uint4& v, float4& p0, float4& p1, int b) {
            v = *(const uint4*)(vrow + 8 * b);
            p0 = *(const float4*)(sc + 8 * b);
            p1 = *(const float4*)(sc + 8 * b + 4);
        };
        auto batch = [&](const uint4& v, const float4& p0, const float4& p1, int b) {
            const float vv[8] = {bf16f(v.x & 0xffffu), bf16f(v.x >> 16), bf16f(v.y & 0xffffu), bf16f(v.y >> 16),
                                 bf16f(v.z & 0xffffu), bf16f(v.z >> 16), bf16f(v.w & 0xffffu), bf16f(v.w >> 16)};
            const float pp[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
            if (b > 0 && 8 * b + 8 <= n) {
#pragma unroll
                for (int j = 0; j < 8; ++j) o = __fmaf_rn(pp[j], vv[j], o);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int t = 8 * b + j;
                    if (t < n) o = t == 0 ? __fmul_rn(pp[j], vv[j]) : __fmaf_rn(pp[j], vv[j], o);
                }
            }
        };
        fetch(va, pa0, pa1, 0);
        for (int b = 0; b < nbat; b += 2) {
            fetch(vb, pb0, pb1, min(b + 1, nbat - 1));
            __builtin_amdgcn_sched_barrier(0);
            batch(va, pa0, pa1, b);
            fetch(va, pa0, pa1, min(b + 2, nbat - 1));
            __builtin_amdgcn_sched_barrier(0);
            if (b + 1 < nbat) batch(vb, pb0, pb1, b + 1);
        }
        a.out[h * HD + es * EW + tid] = __fmul_rn(o, red[2 + ATTN_NT / 64]);
    }
}

// End of a step: the greedy token is recorded, the position advances.
__global__ void step_end_kernel(const uint64_t* tok, int* tokens_out, int* pos_p, int* step_p) {
    tokens_out[*step_p] = (int)*tok;
    *pos_p += 1;
    *step_p += 1;
}

#define GD_HIP(expr)                                                                       \
    do {                                                                                   \
        hipError_t e_ = (expr);                                                            \
        if (e_ != hipSuccess) {                                                            \
            m->err = std::string(#expr) + ": " + hipGetErrorString(e_);                    \
            return 1;                                                                      \
        }                                                                                  \
    } while (0)

// Weight-load slots of the fused matmuls: at least the rows' groups.
template <bool FIRST>
static void launch_qkv(const QkvArgs& a, int ngp, int wgs, hipStream_t st) {
    if (ngp <= 4)
        qkv_kernel<4, FIRST><<<wgs, QKV_NT, 0, st>>>(a);
    else if (ngp <= 6)
        qkv_kernel<6, FIRST><<<wgs, QKV_NT, 0, st>>>(a);
    else
        qkv_kernel<8, FIRST><<<wgs, QKV_NT, 0, st>>>(a);
}

static void launch_ffn(const FfnArgs& a, int ngp, int wgs, hipStream_t st) {
    if (ngp <= 4)
        ffn_kernel<4><<<wgs, FFN_NT, 0, st>>>(a);
    else if (ngp <= 6)
        ffn_kernel<6><<<wgs, FFN_NT, 0, st>>>(a);
    else
        ffn_kernel<8><<<wgs, FFN_NT, 0, st>>>(a);
}

}  // namespace

extern "C" {

struct nngd_model {
    nng_config c;
    std::vector<nnh_weight*> w;  // 7 * n_layer + 1, lm_head (the tied token_embd) last
    std::vector<F32Mat> f;       // the 16-lane layouts of the 7 * n_layer layer weights
    float* norms = nullptr;      // device copy, layout of nng_create
    uint16_t *kc = nullptr, *vc = nullptr;
    float *cos_t = nullptr, *sin_t = nullptr;  // [2][n_ctx][hd/2]: sliding (local) base, then global
    float *xa = nullptr, *xb = nullptr;        // the residual stream, alternating
    float *y = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr, *o = nullptr;
    float *h = nullptr, *logits = nullptr, *record = nullptr;
    void* work = nullptr;
    uint64_t* tok = nullptr;
    int *pos = nullptr, *step = nullptr, *tokens = nullptr;
    int n_gen_max = 0;
    hipStream_t st = nullptr;
    hipGraphExec_t exec = nullptr;
    std::string err;
};

static size_t norm_stride(const nng_config& c) { return 4 * (size_t)c.n_embd + 2 * (size_t)c.head_dim; }

const char* nngd_error(nngd_model* m) { return m->err.c_str(); }

void nngd_free(nngd_model* m) {
    if (!m) return;
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    void* bufs[] = {m->norms, m->kc, m->vc, m->cos_t, m->sin_t, m->xa, m->xb, m->y, m->q, m->k, m->v, m->attn, m->o,
                    m->h, m->logits, m->record, m->work, m->tok, m->pos, m->step, m->tokens};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    if (m->st) (void)hipStreamDestroy(m->st);
    delete m;
}

// RoPE tables exactly as gemma3.cpp's rope_neox forms them: ratio =
// pow(base, -2 / n_rot) and inv *= ratio in f32, theta = pos * inv.
static void rope_table(float base, int n_ctx, int hd, float* cs, float* sn) {
    const int half = hd / 2;
    const float ratio = std::pow(base, -2.0f / (float)hd);
    for (int p = 0; p < n_ctx; ++p) {
        float inv = 1.0f;
        for (int i = 0; i < half; ++i) {
            const float theta = (float)p * inv;
            cs[(size_t)p * half + i] = std::cos(theta);
            sn[(size_t)p * half + i] = std::sin(theta);
            inv *= ratio;
        }
    }
}

int nngd_create(const nng_config* cfg, const float* norms, nnh_weight* const* weights, int n_weights, int n_gen_max,
                nngd_model** out) {
    nngd_model* m = new nngd_model();
    *out = m;
    m->c = *cfg;
    const nng_config& c = m->c;
    if (c.n_ctx > ATTN_BLOCK) {
        m->err = "the device decode holds one attention block: n_ctx <= 256";
        return 1;
    }
    if (n_weights != 7 * c.n_layer + 1 || c.n_head % c.n_kv != 0) {
        m->err = "bad weight count or head grouping";
        return 1;
    }
    if (c.n_embd % 128 || c.n_embd > E_MAX || (c.head_dim != 128 && c.head_dim != 256) || c.n_ff % 32) {
        m->err = "the fused step needs n_embd a multiple of 128 up to 2048, head_dim 128 or 256";
        return 1;
    }
    m->w.assign(weights, weights + n_weights);
    // The fused kernels read q, k, v, gate and up in the 16-lane Q8_0 layout.
    for (int i = 0; i < 7 * c.n_layer; ++i) {
        nnh_f32_layout l;
        if (nnh_weight_f32_layout(weights[i], &l)) {
            m->err = std::string("weight layout: ") + nnh_last_error();
            return 1;
        }
        const int kind = i % 7;
        if (kind != 3 && kind != 6 && (l.dtype != NNH_Q8_0 || l.cols != (size_t)c.n_embd)) {
            m->err = "the fused q, k, v, gate and up matmuls take Q8_0 weights of n_embd columns";
            return 1;
        }
        m->f.push_back(F32Mat{(const uint8_t*)l.quants, l.scales, l.biases, (int)l.rows, (int)l.nb, (int)l.nbp});
    }
    // The lm_head's layouts too, before any step is captured.
    if (nnh_weight_prepare(m->w.back(), NNH_ACT_F32, 1)) {
        m->err = std::string("lm_head layout: ") + nnh_last_error();
        return 1;
    }
    m->n_gen_max = n_gen_max;
    const size_t E = c.n_embd, hd = c.head_dim, qd = (size_t)c.n_head * hd, kvd = (size_t)c.n_kv * hd;
    const size_t nn = norm_stride(c) * c.n_layer + E, half = hd / 2;
    GD_HIP(hipStreamCreateWithFlags(&m->st, hipStreamNonBlocking));
    GD_HIP(hipMalloc((void**)&m->norms, nn * 4));
    GD_HIP(hipMemcpy(m->norms, norms, nn * 4, hipMemcpyHostToDevice));
    GD_HIP(hipMalloc((void**)&m->kc, (size_t)c.n_layer * c.n_ctx * kvd * 2));
    GD_HIP(hipMalloc((void**)&m->vc, (size_t)c.n_layer * c.n_ctx * kvd * 2));
    std::vector<float> cs(2 * (size_t)c.n_ctx * half), sn(2 * (size_t)c.n_ctx * half);
    rope_table(c.rope_base_swa, c.n_ctx, (int)hd, cs.data(), sn.data());
    rope_table(c.rope_base, c.n_ctx, (int)hd, cs.data() + (size_t)c.n_ctx * half, sn.data() + (size_t)c.n_ctx * half);
    GD_HIP(hipMalloc((void**)&m->cos_t, cs.size() * 4));
    GD_HIP(hipMalloc((void**)&m->sin_t, sn.size() * 4));
    GD_HIP(hipMemcpy(m->cos_t, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    GD_HIP(hipMemcpy(m->sin_t, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
    GD_HIP(hipMalloc((void**)&m->xa, E * 4));
    GD_HIP(hipMalloc((void**)&m->xb, E * 4));
    GD_HIP(hipMalloc((void**)&m->y, E * 4));
    GD_HIP(hipMalloc((void**)&m->o, E * 4));
    GD_HIP(hipMalloc((void**)&m->q, qd * 4));
    GD_HIP(hipMalloc((void**)&m->k, kvd * 4));
    GD_HIP(hipMalloc((void**)&m->v, kvd * 4));
    GD_HIP(hipMalloc((void**)&m->attn, qd * 4));
    GD_HIP(hipMalloc((void**)&m->h, (size_t)c.n_ff * 4));
    GD_HIP(hipMalloc((void**)&m->logits, (size_t)c.n_vocab * 4));
    GD_HIP(hipMalloc((void**)&m->record, (size_t)n_gen_max * c.n_layer * E * 4));
    GD_HIP(hipMalloc(&m->work, nnh_model_argmax_work_bytes(m->w.back())));
    GD_HIP(hipMalloc((void**)&m->tok, 8));
    GD_HIP(hipMalloc((void**)&m->pos, 4));
    GD_HIP(hipMalloc((void**)&m->step, 4));
    GD_HIP(hipMalloc((void**)&m->tokens, (size_t)n_gen_max * 4));
    return 0;
}

// Queue one decode step on m->st (eagerly, or into a graph being captured).
static int queue_step(nngd_model* m) {
    const nng_config& c = m->c;
    const int E = c.n_embd, hd = c.head_dim, H = c.n_head, KV = c.n_kv, F = c.n_ff, ngp = (E / 32 + 7) / 8;
    const size_t ns = norm_stride(c), rs = (size_t)c.n_layer * E;
    hipStream_t st = m->st;
    const uint8_t* te = (const uint8_t*)nnh_weight_device_data(m->w.back());
    const float eps = c.rms_eps;
    for (int li = 0; li < c.n_layer; ++li) {
        const float* nr = m->norms + ns * li;
        const float *attn_norm = nr, *q_norm = nr + E, *k_norm = nr + E + hd, *post_attn = nr + E + 2 * hd,
                    *ffn_norm = nr + 2 * E + 2 * hd;
        const bool sliding = c.swa_period > 0 && (li + 1) % c.swa_period != 0;  // load.rs:1156-1160
        const size_t half = hd / 2, tab = sliding ? 0 : (size_t)c.n_ctx * half;
        const F32Mat* f = m->f.data() + 7 * li;
        nnh_weight* const* w = m->w.data() + 7 * li;
        const size_t kvd = (size_t)KV * hd, cache = (size_t)li * c.n_ctx * kvd;
        // The previous layer's post-FFW residual (or the embedding), attention's norm, q / k / v.
        QkvArgs qa{};
        int wgs = 0;
        float* outs[3] = {m->q, m->k, m->v};
        for (int j = 0; j < 3; ++j) {
            qa.m[j] = f[j];
            qa.y[j] = outs[j];
            qa.wg[j] = (f[j].rows + QKV_NT / 16 - 1) / (QKV_NT / 16);
            wgs += qa.wg[j];
        }
        qa.norm = attn_norm;
        qa.x_out = m->xa;
        qa.E = E;
        qa.eps = eps;
        if (li == 0) {
            qa.tok = m->tok;
            qa.tq = (const int8_t*)te;
            qa.ts = (const uint16_t*)(te + (size_t)c.n_vocab * E);
            qa.embd_scale = std::sqrt((float)E);
            launch_qkv<true>(qa, ngp, wgs, st);
        } else {
            qa.o = m->o;
            qa.x_in = m->xb;
            qa.post = m->norms + ns * (li - 1) + 3 * E + 2 * hd;
            qa.rec = m->record + (size_t)(li - 1) * E;
            qa.step_p = m->step;
            qa.rec_stride = rs;
            launch_qkv<false>(qa, ngp, wgs, st);
        }
        AttnArgs aa{m->q,  m->k,         m->v,         q_norm, k_norm, m->cos_t + tab, m->sin_t + tab, m->pos,
                    m->kc + cache, m->vc + cache, H / KV, KV, sliding ? c.window : 0, c.attn_scale, eps, m->attn};
        if (hd == 256)
            attn_kernel<256><<<H * ATTN_SPLIT, ATTN_NT, 0, st>>>(aa);
        else
            attn_kernel<128><<<H * ATTN_SPLIT, ATTN_NT, 0, st>>>(aa);
        if (nnh_gemv_batch_dev(w[3], m->attn, H * hd, m->o, E, 1, NNH_ACT_F32, st)) {
            m->err = std::string("gemv: ") + nnh_last_error();
            return 1;
        }
        FfnArgs fa{f[4], f[5], m->h, F, m->o, m->xa, post_attn, ffn_norm, m->xb, E, eps};
        launch_ffn(fa, ngp, (F + FFN_NT / 32 - 1) / (FFN_NT / 32), st);
        if (nnh_gemv_batch_dev(w[6], m->h, F, m->o, E, 1, NNH_ACT_F32, st)) {
            m->err = std::string("gemv: ") + nnh_last_error();
            return 1;
        }
    }
    // The last residual and y = RMSNorm(x, output_norm); the greedy token is the lm_head argmax of y.
    FinalArgs fin{m->o,    m->xb,   m->norms + ns * (c.n_layer - 1) + 3 * E + 2 * hd, m->norms + ns * c.n_layer,
                  m->xa,   m->y,    m->record + (size_t)(c.n_layer - 1) * E,          m->step,
                  rs,      E,       eps};
    final_kernel<<<1, WG, 0, st>>>(fin);
    if (nnh_model_argmax_dev(m->w.back(), m->y, m->logits, m->work, m->tok, st)) {
        m->err = std::string("lm_head: ") + nnh_last_error();
        return 1;
    }
    step_end_kernel<<<1, 1, 0, st>>>(m->tok, m->tokens, m->pos, m->step);
    GD_HIP(hipGetLastError());
    return 0;
}

// Continue a decode after the CPU harness's prefill: take its KV caches and
// position, then generate: out_tokens[0] = first_token and n_gen - 1
// forwards, as nng_generate's loop does. record gets each forward's
// per-layer hidden states ([n_gen - 1][n_layer][n_embd]); seconds the decode
// wall time.
int nngd_decode(nngd_model* m, nng_model* cpu, int32_t first_token, int n_gen, int32_t* out_tokens, float* record,
                double* seconds) {
    const nng_config& c = m->c;
    if (n_gen < 1 || n_gen - 1 > m->n_gen_max) {
        m->err = "n_gen out of range";
        return 1;
    }
    const uint16_t *kc, *vc;
    size_t pos;
    nng_state(cpu, &kc, &vc, &pos, nullptr, nullptr);
    if (pos + (size_t)n_gen > (size_t)c.n_ctx) {
        m->err = "context full";
        return 1;
    }
    const size_t cache = (size_t)c.n_layer * c.n_ctx * c.n_kv * c.head_dim * 2;
    GD_HIP(hipMemcpy(m->kc, kc, cache, hipMemcpyHostToDevice));
    GD_HIP(hipMemcpy(m->vc, vc, cache, hipMemcpyHostToDevice));
    const uint64_t tok = (uint64_t)first_token;
    const int p = (int)pos, zero = 0;
    GD_HIP(hipMemcpy(m->tok, &tok, 8, hipMemcpyHostToDevice));
    GD_HIP(hipMemcpy(m->pos, &p, 4, hipMemcpyHostToDevice));
    GD_HIP(hipMemcpy(m->step, &zero, 4, hipMemcpyHostToDevice));
    out_tokens[0] = first_token;
    const int steps = n_gen - 1;
    auto t0 = std::chrono::steady_clock::now();
    if (steps > 0) {
        // Step 0 eagerly; it also settles every lazily sized buffer before capture.
        if (queue_step(m)) return 1;
        GD_HIP(hipStreamSynchronize(m->st));
        if (steps > 1) {
            if (!m->exec) {
                hipGraph_t graph;
                GD_HIP(hipStreamBeginCapture(m->st, hipStreamCaptureModeThreadLocal));
                const int rc = queue_step(m);
                hipError_t e = hipStreamEndCapture(m->st, &graph);
                if (rc) return 1;
                GD_HIP(e);
                GD_HIP(hipGraphInstantiate(&m->exec, graph, nullptr, nullptr, 0));
                GD_HIP(hipGraphDestroy(graph));
            }
            for (int s = 1; s < steps; ++s) GD_HIP(hipGraphLaunch(m->exec, m->st));
        }
        GD_HIP(hipStreamSynchronize(m->st));
    }
    auto t1 = std::chrono::steady_clock::now();
    if (seconds) *seconds = std::chrono::duration<double>(t1 - t0).count();
    if (steps > 0) {
        GD_HIP(hipMemcpy(out_tokens + 1, m->tokens, (size_t)steps * 4, hipMemcpyDeviceToHost));
        if (record)
            GD_HIP(hipMemcpy(record, m->record, (size_t)steps * c.n_layer * c.n_embd * 4, hipMemcpyDeviceToHost));
    }
    return 0;
}

}  // extern "C"
