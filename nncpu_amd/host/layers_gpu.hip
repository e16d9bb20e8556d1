// The forward of gemma3.cpp (nng_forward: crates/nncpu/src/model/forward.rs
// 197-439 attention, 719-841 layer, 848-965 model_forward) on the GPU, for
// any number of tokens and any of its architectures (Gemma-3, Llama,
// Qwen2, Qwen3): every weight matmul through the library (nnh_gemv_batch_dev, in
// any activation mode), everything between the matmuls as the kernels
// below, each value computed by the CPU restatement's operations in its
// order and rounding (-ffp-contract=off; __f*_rn where it matters). With
// the bit-exact f32 matmul the hidden states, the K/V cache and the tokens
// equal the CPU forward's bit for bit; with an int8 mode the matmuls carry
// that mode's tolerance and the rest is still the CPU's arithmetic.
//
// Per layer, on one stream (activations [token][dim], f32):
//   qkv         = W_qkv normed (one fused matrix, or q, k, v into column
//                 ranges of one buffer)
//   qkv_post    biases (Qwen2), per-head q / k RMSNorm (Gemma), RoPE from a
//               host table per position, K / V rows appended to the BF16
//               cache, q kept in place
//   attn_part   a partial (o, m, l) per (token, KV head, 256-key block): the
//               scores as 8-lane FMA chains, the block's first maximum,
//               exp_lane weights and their 8-lane sum, the V rows' weighted
//               sum (scalar.rs:444-519)
//   attn_merge  the partials merged in block order with glibc's expf, each
//               head's output divided by its weight sum (scalar.rs:521-548)
//   (one token: qkv_post's work runs inside the attention kernel, and when
//   the grid is one 256-key block so does the merge: one launch for all three)
//   r           = W_o attn
//   resid_norm  x += post_attention_norm(r) (Gemma) or r; normed = ffn_norm(x)
//   gu          = [W_gate; W_up] normed (fused, or gate and up into halves)
//   act         gate = gelu(gate) * up (Gemma) or silu(gate) * up, in place
//   r           = W_down gate
//   resid_norm  x += post_ffw_norm(r) or r, the last token's x recorded as
//               the layer's state; normed = the next layer's attn_norm(x),
//               after the last layer x = output_norm(x)
// The sums of squares of the norms are the CPU's 8 FMA lanes over whole
// 8-chunks (one lane each), hsum8 and an f64 tail; the norm scale is f64.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "gemma3.h"
#include "nncpu_hip.h"
#include "ops_dev.h"
#include "q8_act.h"
#include "rmsnorm_exact.h"

namespace {

constexpr int ATTN_BLOCK = 256;  // model/mod.rs:84-87
constexpr int LDS_MAX = 160 * 1024;

// hsum8 of lanes 0..7's values (valid at lane 0 of each aligned group of 8):
// xor-4 gives v_l + v_{l+4}, xor-1 and xor-2 then add those pairs as hsum8 does.
__device__ __forceinline__ float hsum8_lanes(float a) {
    const float p = __fadd_rn(a, __shfl_xor(a, 4, 64));
    const float q = __fadd_rn(p, __shfl_xor(p, 1, 64));
    return __fadd_rn(q, __shfl_xor(q, 2, 64));
}

__device__ __forceinline__ float hsum8(const float* a) {
    return __fadd_rn(__fadd_rn(__fadd_rn(a[0], a[4]), __fadd_rn(a[1], a[5])),
                     __fadd_rn(__fadd_rn(a[2], a[6]), __fadd_rn(a[3], a[7])));
}

// sum_sq (scalar.rs:232-250) of v[0..dim) (LDS), run by one wave
// (rmsnorm_exact.h); the result is returned to every lane.
__device__ __forceinline__ double row_sumsq(const float* v, int dim, int lane) { return nnh::rms_sumsq(v, dim, lane); }

// A matmul's one-row input written by the kernel that produces it, in the
// library's int8 activation layout (nnh_act_layout_ex, NNH_ACT_I8, one row):
// quants [cols], BF16 block scales [cols / 32], then (scale, scale * sum of
// the block's quants) per block as f64. The values are nncpu's Q8_0 encoder
// (q8_act.h, the library quantizer's own steps), so the bits are those of
// quantizing the f32 row afterwards. q == NULL: nothing is written.
struct QOut {
    int8_t* q;
    uint16_t* s;
    double* sx;
};

using nnh::dpp_f;
using nnh::dpp_i;
using nnh::max8;
using nnh::sum8;

// A thread's pieces of the row into qo (nnh::q8_pieces: piece k is values
// 4i .. 4i+3, i = i0 + k * stride; every lane of the wave calls it).
template <int K>
__device__ __forceinline__ void q8_pieces(const float4 (&p)[K], int i0, int stride, int n4, const QOut& qo) {
    nnh::q8_pieces<K>(p, i0, stride, n4, [&](int i, uint32_t word, const nnh::Q8Scale& s, int qs) {
        ((uint32_t*)qo.q)[i] = word;
        if ((i & 7) == 0) {
            const int b = i >> 3;
            qo.s[b] = (uint16_t)s.bits;
            qo.sx[2 * b] = (double)s.scale;
            qo.sx[2 * b + 1] = (double)s.scale * (double)qs;  // exact: s_x * sum(q_x)
        }
    });
}

// Value j of the row, a block being one half-wave (j & 31 == lane & 31, all
// 32 lanes active).
__device__ __forceinline__ void q8_value(float v, int j, const QOut& qo) {
    float a = max8(nnh::q8_abs(v));
    a = fmaxf(a, dpp_f<0x140>(a));
    a = fmaxf(a, __shfl_xor(a, 16, 64));
    const nnh::Q8Scale s = nnh::q8_scale(a);
    const int q = nnh::q8_quant(v, s.inv);
    int qs = sum8(q);
    qs += dpp_i<0x140>(qs);
    qs += __shfl_xor(qs, 16, 64);
    qo.q[j] = (int8_t)q;
    if ((j & 31) == 0) {
        const int b = j >> 5;
        qo.s[b] = (uint16_t)s.bits;
        qo.sx[2 * b] = (double)s.scale;
        qo.sx[2 * b + 1] = (double)s.scale * (double)qs;
    }
}

// Embedding rows (gemma3.cpp embed_row, kernels/mod.rs:917-954): token t's
// row of the split-layout table times `scale` into x[t].
__global__ void embed_kernel(const int32_t* __restrict__ tok, const uint8_t* __restrict__ table, int wtype,
                             int n_vocab, int E, float scale, float* __restrict__ x) {
    const int t = blockIdx.x;
    int id = tok[t];
    id = id < 0 ? 0 : (id >= n_vocab ? n_vocab - 1 : id);  // the host checks; a device caller gets a clamp
    const size_t te = (size_t)n_vocab * E, nbe = E / 32;
    float* y = x + (size_t)t * E;
    for (int i = threadIdx.x; i < E; i += blockDim.x) {
        const int b = i >> 5, k = i & 31;
        if (wtype == 2) {
            const uint8_t* tq = table + (size_t)id * (E / 2);
            const uint16_t* ts = (const uint16_t*)(table + te / 2) + (size_t)id * nbe;
            const uint16_t* tb = (const uint16_t*)(table + te / 2 + te / 16) + (size_t)id * nbe;
            const float s = __fmul_rn(bf16f(ts[b]), scale), bias = __fmul_rn(bf16f(tb[b]), scale);
            const uint8_t q = tq[16 * b + (k & 15)];
            y[i] = __fadd_rn(__fmul_rn(s, (float)(k < 16 ? q & 15 : q >> 4)), bias);
        } else {
            const int8_t* tq = (const int8_t*)table + (size_t)id * E;
            const uint16_t* ts = (const uint16_t*)(table + te) + (size_t)id * nbe;
            y[i] = __fmul_rn((float)tq[i], __fmul_rn(bf16f(ts[b]), scale));
        }
    }
}

// One workgroup of 256 threads per row (dim a multiple of 4, at most 8192):
//   r == NULL: y = rmsnorm(x) * gamma (y may be x);
//   else: x += (post ? rmsnorm(r) * post : r), written back, the last row's
//   new x copied to rec (if not NULL), then y = rmsnorm(x) * gamma (y may be x);
//   qo.q != NULL (one row, dim a multiple of 32): y also quantized into qo.
// rmsnorm_gamma_multi (scalar.rs:270-292): y = (x * scale) * gamma. Every
// thread loads its 16-byte pieces at once; the sums of squares are the 8
// FMA lanes of wave 0 over the row in LDS.
// RN_K: 16-byte pieces per thread, the fewest of 1, 2, 4, 8 that cover the
// row (launch_resid_norm), so no thread carries empty pieces through the
// norm or the quantizer.
constexpr int RN_T = 256;  // threads
template <int RN_K>
__global__ __launch_bounds__(RN_T) void resid_norm_kernel(float* x, const float* __restrict__ r,
                                                          const float* __restrict__ post, const float* gamma,
                                                          float* y, float* __restrict__ rec, int n_rows, int dim,
                                                          float eps, QOut qo) {
    extern __shared__ __align__(16) float lds[];
    __shared__ float scale_s;
    float* v = lds;        // the row being normed
    float* w = lds + dim;  // r, when it is normed first
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, n4 = dim / 4;
    float4* xr = (float4*)(x + (size_t)row * dim);
    float4 xv[RN_K], rv[RN_K], pv[RN_K], gv[RN_K];
#pragma unroll
    for (int k = 0; k < RN_K; ++k) {
        const int i = tid + k * RN_T;
        if (i < n4) {
            xv[k] = xr[i];
            gv[k] = ((const float4*)gamma)[i];
            if (r) rv[k] = ((const float4*)(r + (size_t)row * dim))[i];
            if (post) pv[k] = ((const float4*)post)[i];
        }
    }
    if (r) {
        float sc = 1.0f;
        if (post) {
#pragma unroll
            for (int k = 0; k < RN_K; ++k)
                if (tid + k * RN_T < n4) ((float4*)w)[tid + k * RN_T] = rv[k];
            __syncthreads();
            if (tid < 64) {
                const double ss = row_sumsq(w, dim, lane);
                if (lane == 0) scale_s = rms_of_d(ss, dim, eps);
            }
            __syncthreads();
            sc = scale_s;
        }
#pragma unroll
        for (int k = 0; k < RN_K; ++k) {
            const int i = tid + k * RN_T;
            if (i < n4) {
                float4 nv;
                if (post) {
                    nv.x = __fadd_rn(xv[k].x, __fmul_rn(__fmul_rn(rv[k].x, sc), pv[k].x));
                    nv.y = __fadd_rn(xv[k].y, __fmul_rn(__fmul_rn(rv[k].y, sc), pv[k].y));
                    nv.z = __fadd_rn(xv[k].z, __fmul_rn(__fmul_rn(rv[k].z, sc), pv[k].z));
                    nv.w = __fadd_rn(xv[k].w, __fmul_rn(__fmul_rn(rv[k].w, sc), pv[k].w));
                } else {
                    nv.x = __fadd_rn(xv[k].x, rv[k].x);
                    nv.y = __fadd_rn(xv[k].y, rv[k].y);
                    nv.z = __fadd_rn(xv[k].z, rv[k].z);
                    nv.w = __fadd_rn(xv[k].w, rv[k].w);
                }
                xv[k] = nv;
                xr[i] = nv;
                if (rec && row == n_rows - 1) ((float4*)rec)[i] = nv;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < RN_K; ++k)
        if (tid + k * RN_T < n4) ((float4*)v)[tid + k * RN_T] = xv[k];
    __syncthreads();
    if (tid < 64) {
        const double ss = row_sumsq(v, dim, lane);
        if (lane == 0) scale_s = rms_of_d(ss, dim, eps);
    }
    __syncthreads();
    const float sc = scale_s;
    float4* yr = (float4*)(y + (size_t)row * dim);
    float4 o[RN_K];
#pragma unroll
    for (int k = 0; k < RN_K; ++k) {
        const int i = tid + k * RN_T;
        o[k] = float4{0.0f, 0.0f, 0.0f, 0.0f};
        if (i < n4) {
            o[k].x = __fmul_rn(__fmul_rn(xv[k].x, sc), gv[k].x);
            o[k].y = __fmul_rn(__fmul_rn(xv[k].y, sc), gv[k].y);
            o[k].z = __fmul_rn(__fmul_rn(xv[k].z, sc), gv[k].z);
            o[k].w = __fmul_rn(__fmul_rn(xv[k].w, sc), gv[k].w);
            yr[i] = o[k];
        }
    }
    if (qo.q) q8_pieces<RN_K>(o, tid, RN_T, n4, qo);
}

static void launch_resid_norm(float* x, const float* r, const float* post, const float* gamma, float* y,
                              float* rec, int n_rows, int dim, float eps, QOut qo, hipStream_t st) {
    const size_t lds = (size_t)dim * (r && post ? 8 : 4);
    const int pieces = (dim / 4 + RN_T - 1) / RN_T;
    if (pieces <= 1)
        resid_norm_kernel<1><<<n_rows, RN_T, lds, st>>>(x, r, post, gamma, y, rec, n_rows, dim, eps, qo);
    else if (pieces <= 2)
        resid_norm_kernel<2><<<n_rows, RN_T, lds, st>>>(x, r, post, gamma, y, rec, n_rows, dim, eps, qo);
    else if (pieces <= 4)
        resid_norm_kernel<4><<<n_rows, RN_T, lds, st>>>(x, r, post, gamma, y, rec, n_rows, dim, eps, qo);
    else
        resid_norm_kernel<8><<<n_rows, RN_T, lds, st>>>(x, r, post, gamma, y, rec, n_rows, dim, eps, qo);
}

struct QkvArgs {
    float* qkv;              // [n_tok][QKV]: q, k, v
    const float* bias;       // [QKV] of this layer, or NULL
    const float* qn;         // per-head q / k RMSNorm gammas (Gemma), or NULL
    const float* kn;
    const float* cs;         // RoPE table of this layer's base: [n_ctx][hd / 2]
    const float* sn;
    uint16_t* kc;            // this layer's cache rows: [n_ctx][KVD]
    uint16_t* vc;
    const int* posp;         // the first token's position in device memory, or NULL: pos0
    int H, KV, hd, QKV, pos0, rope_mode, n_ctx;
    float eps;
};

// One wave per (token, head slot): q heads, then k heads, then v heads
// (forward.rs:255-351 for one head's values, in the CPU restatement's order:
// bias, norm, RoPE, then the BF16 append).
__global__ __launch_bounds__(64) void qkv_post_kernel(QkvArgs a) {
    extern __shared__ float v[];
    const int t = blockIdx.x, s = blockIdx.y, lane = threadIdx.x, hd = a.hd;
    const int kind = s < a.H ? 0 : (s < a.H + a.KV ? 1 : 2), head = kind == 0 ? s : (kind == 1 ? s - a.H : s - a.H - a.KV);
    const int off = kind == 0 ? head * hd : a.H * hd + (kind - 1) * a.KV * hd + head * hd;
    float* src = a.qkv + (size_t)t * a.QKV + off;
    for (int i = lane; i < hd; i += 64) v[i] = a.bias ? __fadd_rn(src[i], a.bias[off + i]) : src[i];
    __syncthreads();
    if (kind < 2) {
        const float* g = kind == 0 ? a.qn : a.kn;
        if (g) {
            const float sc = rms_of_d(row_sumsq(v, hd, lane), hd, a.eps);
            __syncthreads();
            for (int i = lane; i < hd; i += 64) v[i] = __fmul_rn(__fmul_rn(v[i], sc), g[i]);
            __syncthreads();
        }
        const int half = hd / 2, pos = (a.posp ? *a.posp : a.pos0) + t;
        const int stride = a.rope_mode == NNG_ROPE_NORM ? 2 : 1, partner = a.rope_mode == NNG_ROPE_NORM ? 1 : half;
        const int pr = pos < a.n_ctx ? pos : a.n_ctx - 1;
        const float* cs = a.cs + (size_t)pr * half;
        const float* sn = a.sn + (size_t)pr * half;
        for (int i = lane; i < half; i += 64) {
            const int p = i * stride;
            const float x0 = v[p], x1 = v[p + partner], c = cs[i], sv = sn[i];
            v[p] = __fsub_rn(__fmul_rn(c, x0), __fmul_rn(sv, x1));
            v[p + partner] = __fadd_rn(__fmul_rn(sv, x0), __fmul_rn(c, x1));
        }
        __syncthreads();
    }
    const int pos = (a.posp ? *a.posp : a.pos0) + t;
    if (kind == 0) {
        for (int i = lane; i < hd; i += 64) src[i] = v[i];
    } else if (pos < a.n_ctx) {  // a device position past the context writes nothing
        uint16_t* dst = (kind == 1 ? a.kc : a.vc) + (size_t)pos * a.KV * hd + head * hd;
        for (int i = lane; i < hd; i += 64) dst[i] = to_bf16(v[i]);
    }
}

struct AttnArgs {
    const float* qkv;        // q of every token at [t][QKV]
    const uint16_t* kc;      // this layer's cache: [n_ctx][KVD] BF16
    const uint16_t* vc;
    float* parts;            // [n_tok][KV][nblk][G][hd + 2]
    float* out;              // [n_tok][H * hd]
    const uint64_t* expt;    // glibc_expf's table
    const int* posp;         // the first token's position in device memory, or NULL: pos0
    int KV, G, hd, QKV, nblk, pos0, n_seq, window, n_tok, tq, n_ctx;
    float scale;
};

// The batch's first position and the sequence length after it (both from
// device memory for a replayed decode step), the length capped at the
// context so no read leaves the cache.
__device__ __forceinline__ void attn_pos(const AttnArgs& a, int& p0, int& n_seq) {
    p0 = a.posp ? *a.posp : a.pos0;
    n_seq = a.posp ? p0 + a.n_tok : a.n_seq;
    n_seq = n_seq < a.n_ctx ? n_seq : a.n_ctx;
}

// model/embed.rs:14-30, the causal branch (gemma3.cpp attn_span).
__device__ __forceinline__ void attn_span(int window, int pos, int n_seq, int& first, int& last) {
    const int end = n_seq ? n_seq - 1 : 0;
    first = (window > 0 && pos + 1 > window) ? pos + 1 - window : 0;
    last = pos < end ? pos : end;
}

// Token t's keys in 256-key block b (false when its span has none), and
// the index of b among its span's blocks.
__device__ __forceinline__ bool tok_block(const AttnArgs& a, int p0, int n_seq, int t, int b, int& k0, int& k1,
                                          int& bi) {
    if (t >= a.n_tok) return false;
    int first, last;
    attn_span(a.window, p0 + t, n_seq, first, last);
    if (b < first / ATTN_BLOCK || b > last / ATTN_BLOCK) return false;
    k0 = first > b * ATTN_BLOCK ? first : b * ATTN_BLOCK;
    k1 = last < b * ATTN_BLOCK + ATTN_BLOCK - 1 ? last : b * ATTN_BLOCK + ATTN_BLOCK - 1;
    bi = b - first / ATTN_BLOCK;
    return true;
}

// The partials (scalar.rs:444-519, gemma3.cpp attn_block) of tokens
// x * tq .. + tq - 1, heads of KV head y, over 256-key block z: rows
// r = s * G + h (token slot s, head h), at most AT_NQ. Every row's values
// are the CPU's: its scores, first maximum, weights, weight sum and V sum
// over the token's own keys of the block, in key order. The workgroup stages
// the block's K rows (then V rows) AT_KC at a time in LDS for all its rows.
// Scores: thread (key j, half) holds K row j in registers and runs the
// 8-lane FMA chains of its half's rows, the queries (the same for the whole
// wave) read by scalar loads. V sums: thread (columns, row group) keeps the
// chains o[r][i] of its rows and columns across the chunks. The LDS moves
// about 4 bytes per FMA lane when the wave-uniform operand comes from LDS
// (a broadcast read still returns 64 lanes' data), half the VALU's rate:
// hence scalar queries, and several columns per weight read.
constexpr int AT_KC = 128;  // keys per LDS chunk
constexpr int AT_NQ = 32;   // rows per workgroup at most (16 at head_dim 256: registers)
__host__ __device__ constexpr int at_nq(int hd) { return hd >= 256 ? 16 : AT_NQ; }

template <int HD>
__global__ __launch_bounds__(256) void attn_tile_kernel(AttnArgs a) {
    constexpr int KS = HD + 8;
    static_assert(HD % 8 == 0 && 256 % HD == 0 && HD >= 32, "head_dim 32, 64, 128 or 256");
    extern __shared__ __align__(16) float lds[];
    __shared__ int tk0[AT_NQ], tk1[AT_NQ], tbi[AT_NQ], rk0[AT_NQ], rk1[AT_NQ];
    const int kvh = blockIdx.y, b = blockIdx.z, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = a.G, TQ = a.tq, NQ = TQ * G, t0 = blockIdx.x * TQ, pw = HD + 2, KVD = a.KV * HD;
    // The tile's key range in the block (every thread computes it).
    int p0, n_seq;
    attn_pos(a, p0, n_seq);
    int K0 = 1 << 30, K1 = -1;
    for (int s = 0; s < TQ; ++s) {
        int k0, k1, bi;
        const bool on = tok_block(a, p0, n_seq, t0 + s, b, k0, k1, bi);
        if (tid == 0) {
            tk0[s] = on ? k0 : 1;
            tk1[s] = on ? k1 : 0;
            tbi[s] = bi;
        }
        if (on) {
            K0 = k0 < K0 ? k0 : K0;
            K1 = k1 > K1 ? k1 : K1;
        }
    }
    if (K1 < 0) return;
    __syncthreads();
    if (tid < NQ) {  // each row's key range: its token's
        rk0[tid] = tk0[tid / G];
        rk1[tid] = tk1[tid / G];
    }
    float* sc = lds;                              // [NQ][256], key k at k - K0
    float* mh = sc + NQ * ATTN_BLOCK;             // [AT_NQ]
    uint16_t* kv = (uint16_t*)(mh + AT_NQ);       // [AT_KC][KS]
    __syncthreads();
    // Scores, chunk by chunk.
    constexpr int PR = HD / 8;  // 16-byte pieces per row
    for (int c0 = K0; c0 <= K1; c0 += AT_KC) {
        const int nkc = K1 + 1 - c0 < AT_KC ? K1 + 1 - c0 : AT_KC;
        for (int i = tid; i < nkc * PR; i += 256) {
            const int j = i / PR, c = i - j * PR;
            *(uint4*)(kv + j * KS + 8 * c) = *(const uint4*)(a.kc + (size_t)(c0 + j) * KVD + kvh * HD + 8 * c);
        }
        __syncthreads();
        const int j = tid & (AT_KC - 1), half = tid >> 7;
        if (j < nkc) {
            const int key = c0 + j;
            // The key's row in registers as f32 up to head_dim 128 (converted
            // once for all rows); at 256 it is read from LDS with the queries.
            constexpr bool F32ROW = HD <= 128;
            const uint16_t* krow = kv + j * KS;
            float kf[F32ROW ? HD : 1];
            if (F32ROW) {
#pragma unroll
                for (int c = 0; c < PR; ++c) {
                    const uint4 k8 = *(const uint4*)(krow + 8 * c);
                    const uint32_t kw[4] = {k8.x, k8.y, k8.z, k8.w};
#pragma unroll
                    for (int l = 0; l < 8; ++l)
                        kf[F32ROW ? 8 * c + l : 0] = bf16f((kw[l >> 1] >> (16 * (l & 1))) & 0xffffu);
                }
            }
            // The two halves take token slots (or, with one token per tile,
            // alternate heads). A row's queries are the same for the whole
            // wave: read from global memory at a wave-uniform address (scalar
            // loads; nothing in this kernel writes them), so the FMAs take
            // them as scalar operands and only the K rows come from LDS.
            const int hs = (TQ + 1) / 2;
            const int ts0 = TQ >= 2 ? half * hs : 0, ts1 = TQ >= 2 ? (half + 1) * hs < TQ ? (half + 1) * hs : TQ : 1;
            const int h0 = TQ >= 2 ? 0 : half, hstep = TQ >= 2 ? 1 : 2;
            for (int ts = ts0; ts < ts1; ++ts) {
                if (key < tk0[ts] || key > tk1[ts]) continue;
                for (int h = h0; h < G; h += hstep) {
                    const int r = ts * G + h;
                    const float* __restrict__ qg =
                        a.qkv + (size_t)__builtin_amdgcn_readfirstlane((t0 + ts) * a.QKV + (kvh * G + h) * HD);
                    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int c = 0; c < PR; ++c) {
                        float qv[8];
#pragma unroll
                        for (int l = 0; l < 8; ++l) qv[l] = qg[8 * c + l];
                        if (F32ROW) {
#pragma unroll
                            for (int l = 0; l < 8; ++l) acc[l] = __fmaf_rn(qv[l], kf[F32ROW ? 8 * c + l : 0], acc[l]);
                        } else {
                            const uint4 k8 = *(const uint4*)(krow + 8 * c);
                            const uint32_t kw[4] = {k8.x, k8.y, k8.z, k8.w};
#pragma unroll
                            for (int l = 0; l < 8; ++l)
                                acc[l] = __fmaf_rn(qv[l], bf16f((kw[l >> 1] >> (16 * (l & 1))) & 0xffffu), acc[l]);
                        }
                    }
                    sc[r * ATTN_BLOCK + key - K0] = __fmul_rn(hsum8(acc), a.scale);
                }
            }
        }
        __syncthreads();
    }
    // Each row's maximum as `if m < v { m = v }` from its first key finds it:
    // the first largest, NaN never taken unless the first score is NaN.
    // Lane l scans keys 4l .. 4l + 3 of the row from -inf, then the lanes'
    // results combine in key order.
    for (int r = wave; r < NQ; r += 4) {
        const int n = rk1[r] + 1 - rk0[r];
        if (n <= 0) continue;
        const float* sr = sc + r * ATTN_BLOCK + (rk0[r] - K0);
        float m = -INFINITY;
        for (int j = 4 * lane; j < 4 * lane + 4 && j < n; ++j)
            if (m < sr[j]) m = sr[j];
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float other = __shfl_xor(m, o, 64);
            const float lo = (lane & o) ? other : m, hi = (lane & o) ? m : other;
            m = lo < hi ? hi : lo;
        }
        if (lane == 0) mh[r] = sr[0] != sr[0] ? sr[0] : m;
    }
    __syncthreads();
    for (int i = tid; i < NQ * ATTN_BLOCK; i += 256) {
        const int r = i >> 8, k = K0 + (i & (ATTN_BLOCK - 1));
        if (k >= rk0[r] && k <= rk1[r]) sc[i] = exp_lane(__fsub_rn(sc[i], mh[r]));
    }
    __syncthreads();
    // The weight sums: lane l of row r's group of 8 adds weights l, l + 8, ..
    // of the row's whole 8-chunks, hsum8, then the tail in order.
    {
        const int r = tid >> 3, l = tid & 7, s = r / G;
        const int n = r < NQ ? rk1[r] + 1 - rk0[r] : 0, body = n & ~7;
        const float* sr = sc + r * ATTN_BLOCK + (r < NQ ? rk0[r] - K0 : 0);
        float vs = 0.0f;
        for (int j = l; j < body; j += 8) vs = __fadd_rn(vs, sr[j]);
        float ls = hsum8_lanes(vs);
        if (n > 0 && l == 0) {
            for (int j = body; j < n; ++j) ls = __fadd_rn(ls, sr[j]);
            const int h = r - s * G;
            float* part = a.parts + ((((size_t)(t0 + s) * a.KV + kvh) * a.nblk) + tbi[s]) * G * pw + h * pw;
            part[HD] = mh[r];
            part[HD + 1] = ls;
        }
    }
    // V sums, chunk by chunk: the first key of a row writes w * v, the rest
    // FMA. Each chain starts at -0, so the first key's FMA is exactly w * v
    // (x + -0 = x for every x, signed zeros included). Thread (row group,
    // column group) runs the chains of CPT adjacent columns of its rows, so
    // each weight read (the same for the whole wave: one row group per wave
    // from head_dim 64) feeds CPT FMAs. Keys every active row of the tile has
    // ([kf0, kf1]) run without masks, four per step, the next step's reads
    // issued before this step's FMAs; keys only some rows have run masked.
    constexpr int CPT = HD >= 64 ? HD / 64 : 1, CG = HD / CPT, RG = 256 / CG;
    constexpr int RPT = (at_nq(HD) + RG - 1) / RG;
    const int cg = tid % CG, rg = tid / CG, ie = cg * CPT;
    float o[RPT][CPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k)
#pragma unroll
        for (int c = 0; c < CPT; ++c) o[k][c] = -0.0f;
    int kf0 = K0, kf1 = K1;
    for (int r = 0; r < NQ; ++r)
        if (rk1[r] >= rk0[r]) {
            kf0 = rk0[r] > kf0 ? rk0[r] : kf0;
            kf1 = rk1[r] < kf1 ? rk1[r] : kf1;
        }
    const float* wrow[RPT];  // each row's weights, indexed by key (rows past NQ read row NQ - 1)
#pragma unroll
    for (int k = 0; k < RPT; ++k) wrow[k] = sc + (rg + RG * k < NQ ? rg + RG * k : NQ - 1) * ATTN_BLOCK - K0;
    // CPT BF16 values of one V row at the thread's columns.
    auto vload = [&](int j, float* v) {
        const uint16_t* p = kv + j * KS + ie;
        if (CPT == 1) {
            v[0] = bf16f(p[0]);
        } else if (CPT == 2) {
            const uint32_t u = *(const uint32_t*)p;
            v[0] = bf16f(u & 0xffffu);
            v[CPT > 1 ? 1 : 0] = bf16f(u >> 16);
        } else {
            const uint2 u = *(const uint2*)p;
            v[0] = bf16f(u.x & 0xffffu);
            v[CPT > 1 ? 1 : 0] = bf16f(u.x >> 16);
            v[CPT > 2 ? 2 : 0] = bf16f(u.y & 0xffffu);
            v[CPT > 3 ? 3 : 0] = bf16f(u.y >> 16);
        }
    };
    for (int c0 = K0; c0 <= K1; c0 += AT_KC) {
        const int nkc = K1 + 1 - c0 < AT_KC ? K1 + 1 - c0 : AT_KC, c1 = c0 + nkc;
        __syncthreads();  // the previous chunk's (or the scores') reads are done
        for (int i = tid; i < nkc * PR; i += 256) {
            const int j = i / PR, c = i - j * PR;
            *(uint4*)(kv + j * KS + 8 * c) = *(const uint4*)(a.vc + (size_t)(c0 + j) * KVD + kvh * HD + 8 * c);
        }
        __syncthreads();
        // The unmasked keys of this chunk, from a multiple of 4 past K0.
        int f0 = kf0 > c0 ? kf0 : c0, f1 = kf1 + 1 < c1 ? kf1 + 1 : c1;
        f0 = K0 + ((f0 - K0 + 3) & ~3);
        if (f1 < f0) f1 = f0;
        f1 = f0 + ((f1 - f0) & ~3);
        auto masked = [&](int key) {
            float v[CPT];
            vload(key - c0, v);
#pragma unroll
            for (int k = 0; k < RPT; ++k) {
                const int r = rg + RG * k < NQ ? rg + RG * k : NQ - 1;
                const bool on = rg + RG * k < NQ && key >= rk0[r] && key <= rk1[r];
                const float w = wrow[k][key];
#pragma unroll
                for (int c = 0; c < CPT; ++c) {
                    const float nv = __fmaf_rn(w, v[c], o[k][c]);
                    o[k][c] = on ? nv : o[k][c];
                }
            }
        };
        for (int key = c0; key < f0 && key < c1; ++key) masked(key);
        if (f0 < f1) {
            // Two register sets used in turn (no copies): a step's FMAs run
            // on one while the next step's reads fill the other.
            float4 wa[RPT], wb[RPT];
            float va[4][CPT], vb[4][CPT];
            auto fetch = [&](int key, float4* w, float (*v)[CPT]) {
#pragma unroll
                for (int k = 0; k < RPT; ++k) w[k] = *(const float4*)(wrow[k] + key);
#pragma unroll
                for (int u = 0; u < 4; ++u) vload(key - c0 + u, v[u]);
            };
            auto step = [&](const float4* w, const float (*v)[CPT]) {
#pragma unroll
                for (int k = 0; k < RPT; ++k) {
                    const float w4[4] = {w[k].x, w[k].y, w[k].z, w[k].w};
#pragma unroll
                    for (int u = 0; u < 4; ++u)
#pragma unroll
                        for (int c = 0; c < CPT; ++c) o[k][c] = __fmaf_rn(w4[u], v[u][c], o[k][c]);
                }
            };
            fetch(f0, wa, va);
            int key = f0;
            for (; key + 8 <= f1; key += 8) {
                fetch(key + 4, wb, vb);
                step(wa, va);
                if (key + 8 < f1) fetch(key + 8, wa, va);
                step(wb, vb);
            }
            if (key < f1) step(wa, va);
        }
        for (int key = f1 > f0 ? f1 : f0; key < c1; ++key)
            if (key >= c0) masked(key);
    }
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        const int r = rg + RG * k;
        if (r >= NQ || rk1[r] < rk0[r]) continue;
        const int s = r / G, h = r - s * G;
        float* dst = a.parts + ((((size_t)(t0 + s) * a.KV + kvh) * a.nblk) + tbi[s]) * G * pw + h * pw + ie;
#pragma unroll
        for (int c = 0; c < CPT; ++c) dst[c] = o[k][c];
    }
}

// Batch u0 .. u0 + U - 1 of a thread's 16-byte pieces of cache rows k0 ..
// k0 + nk - 1 (KV head kvh's HD columns; nk >= 1): every load issued before
// any is used, then stored into LDS rows of HD + 8 halves. Loads and stores
// are unconditional (a conditional store lets the compiler sink its load
// into the branch, one round trip per piece): LDS rows nk .. 255 get copies
// of row nk - 1 and are never read.
template <int HD, int U>
__device__ __forceinline__ void kv_load(uint4 (&r)[U], const uint16_t* __restrict__ src, int k0, int nk, int KVD,
                                        int kvh, int tid, int u0) {
    constexpr int PR = HD / 8;
    // A uniform base and 32-bit offsets: one address register per load.
    const uint16_t* base = src + (size_t)k0 * KVD + kvh * HD;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int i = tid + 256 * (u0 + u), j = i / PR, c = i % PR;
        r[u] = *(const uint4*)(base + (uint32_t)((j < nk ? j : nk - 1) * KVD + 8 * c));
    }
}
template <int HD, int U>
__device__ __forceinline__ void kv_store(const uint4 (&r)[U], uint16_t* kv, int tid, int u0) {
    constexpr int PR = HD / 8, KS = HD + 8;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int i = tid + 256 * (u0 + u), j = i / PR, c = i % PR;
        *(uint4*)(kv + j * KS + 8 * c) = r[u];
    }
}

// Eight keys of a thread's V column (LDS rows of KS halves): the weights and
// the raw BF16 values (converted in fma, so a load waits for nothing), and
// their FMAs into the chain in key order.
struct V8 {
    float4 w0, w1;
    uint32_t v[8];
    template <int KS>
    __device__ __forceinline__ void load(const float* sc, const uint16_t* col, int j) {
        w0 = *(const float4*)(sc + j);
        w1 = *(const float4*)(sc + j + 4);
#pragma unroll
        for (int r = 0; r < 8; ++r) v[r] = col[(j + r) * KS];
    }
    __device__ __forceinline__ float fma(float o) const {
        const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int r = 0; r < 8; ++r) o = __fmaf_rn(w[r], bf16f(v[r]), o);
        return o;
    }
};

// One token's q head `qh` (wave 0) and, when `own`, its key and value rows of
// KV head `kvh` (waves 1 and 2), into rows[0..2][hd] (LDS): qkv_post_kernel's
// operations in its order (bias, per-head RMSNorm, RoPE at position p0, the
// value row with its bias only). Every wave of the workgroup calls it (it
// holds barriers); wave 3 only waits.
template <int HD>
__device__ __forceinline__ void decode_qkv_rows(const QkvArgs& a, float* rows, int qh, int kvh, bool own, int p0,
                                                int wave, int lane) {
    const int kind = wave < 3 ? wave : 3;
    const bool act = kind == 0 || (kind < 3 && own);
    const int off = kind == 0 ? qh * HD : (kind == 1 ? a.H * HD + kvh * HD : a.H * HD + a.KV * HD + kvh * HD);
    float* v = rows + (kind < 3 ? kind : 0) * HD;
    if (act)
        for (int i = lane; i < HD; i += 64) v[i] = a.bias ? __fadd_rn(a.qkv[off + i], a.bias[off + i]) : a.qkv[off + i];
    __syncthreads();
    const float* g = kind == 0 ? a.qn : a.kn;
    if (act && kind < 2 && g) {
        const float sc = rms_of_d(row_sumsq(v, HD, lane), HD, a.eps);
        for (int i = lane; i < HD; i += 64) v[i] = __fmul_rn(__fmul_rn(v[i], sc), g[i]);
    }
    __syncthreads();
    if (act && kind < 2) {
        const int half = HD / 2;
        const int stride = a.rope_mode == NNG_ROPE_NORM ? 2 : 1, partner = a.rope_mode == NNG_ROPE_NORM ? 1 : half;
        const int pr = p0 < a.n_ctx ? p0 : a.n_ctx - 1;
        const float* cs = a.cs + (size_t)pr * half;
        const float* sn = a.sn + (size_t)pr * half;
        for (int i = lane; i < half; i += 64) {
            const int p = i * stride;
            const float x0 = v[p], x1 = v[p + partner], c = cs[i], sv = sn[i];
            v[p] = __fsub_rn(__fmul_rn(c, x0), __fmul_rn(sv, x1));
            v[p + partner] = __fadd_rn(__fmul_rn(sv, x0), __fmul_rn(c, x1));
        }
    }
    __syncthreads();
}

// decode_qkv_rows with its global reads issued first and consumed later, so
// a caller can put further loads (the K/V rows) in flight between them: the
// row's values with their bias and the RoPE coefficients at p0, loaded by
// every lane of every wave unconditionally (a wave without a row rereads the
// q head's; indices clamped), so the waits count them exactly.
template <int HD>
struct QkvRegs {
    static constexpr int NV = (HD + 63) / 64, NR = (HD / 2 + 63) / 64;
    float x[NV], b[NV], c[NR], s[NR];
};
template <int HD>
__device__ __forceinline__ void decode_qkv_issue(const QkvArgs& a, QkvRegs<HD>& g, int qh, int kvh, int p0, int wave,
                                                 int lane) {
    const int kind = wave < 3 ? wave : 0;
    const int off = kind == 0 ? qh * HD : (kind == 1 ? a.H * HD + kvh * HD : a.H * HD + a.KV * HD + kvh * HD);
    const float* bsrc = a.bias ? a.bias : a.qkv;  // a dummy read without biases, unused
#pragma unroll
    for (int k = 0; k < QkvRegs<HD>::NV; ++k) {
        const int i = lane + 64 * k < HD ? lane + 64 * k : HD - 1;
        g.x[k] = a.qkv[off + i];
        g.b[k] = bsrc[off + i];
    }
    const int half = HD / 2, pr = p0 < a.n_ctx ? p0 : a.n_ctx - 1;
#pragma unroll
    for (int k = 0; k < QkvRegs<HD>::NR; ++k) {
        const int i = lane + 64 * k < half ? lane + 64 * k : half - 1;
        g.c[k] = a.cs[(size_t)pr * half + i];
        g.s[k] = a.sn[(size_t)pr * half + i];
    }
}
template <int HD>
__device__ __forceinline__ void decode_qkv_finish(const QkvArgs& a, const QkvRegs<HD>& g, float* rows, bool own,
                                                  int wave, int lane) {
    const int kind = wave < 3 ? wave : 3;
    const bool act = kind == 0 || (kind < 3 && own);
    float* v = rows + kind * HD;
    // Stored by every wave (wave 3 into a row of its own, never read), so the
    // loads' only use is not under a branch the compiler could sink them into.
#pragma unroll
    for (int k = 0; k < QkvRegs<HD>::NV; ++k)
        if (lane + 64 * k < HD) v[lane + 64 * k] = a.bias ? __fadd_rn(g.x[k], g.b[k]) : g.x[k];
    __syncthreads();
    const float* gm = kind == 0 ? a.qn : a.kn;
    if (act && kind < 2 && gm) {
        const float sc = rms_of_d(row_sumsq(v, HD, lane), HD, a.eps);
        for (int i = lane; i < HD; i += 64) v[i] = __fmul_rn(__fmul_rn(v[i], sc), gm[i]);
    }
    __syncthreads();
    if (act && kind < 2) {
        const int half = HD / 2;
        const int stride = a.rope_mode == NNG_ROPE_NORM ? 2 : 1, partner = a.rope_mode == NNG_ROPE_NORM ? 1 : half;
#pragma unroll
        for (int k = 0; k < QkvRegs<HD>::NR; ++k) {
            const int i = lane + 64 * k;
            if (i >= half) continue;
            const int p = i * stride;
            const float x0 = v[p], x1 = v[p + partner], c = g.c[k], sv = g.s[k];
            v[p] = __fsub_rn(__fmul_rn(c, x0), __fmul_rn(sv, x1));
            v[p + partner] = __fadd_rn(__fmul_rn(sv, x0), __fmul_rn(c, x1));
        }
    }
    __syncthreads();
}

// One token's partial (decode) for query head x of KV head y over its block
// b0 + z: attn_tile_kernel's arithmetic for a single row, spread over more
// workgroups (one per head and block) for latency: the block's K and V rows
// staged whole in LDS, together up to head_dim 128 (each thread's loads
// issued at once: one round trip), at 256 V after the scores; thread j the
// score of key j (query by scalar loads), the first maximum and weight sum
// as there, thread i the V chain of column i (from -0, so the first key's
// FMA is w * v exactly). Its LDS (the staged rows) allows at most two
// workgroups per CU, so the registers are budgeted for two waves per SIMD.
//
// qkv_post_kernel's work for the rows this workgroup reads is done here first, by the same operations
// (so the same bits): wave 0 forms the query head (bias, q norm, RoPE) in
// LDS, waves 1 and 2 the token's key and value rows when the token's
// position lies in this workgroup's block (those rows then replace the
// cache's row in the staged copy, and query head 0 of the KV head appends
// them to the cache as BF16). With `direct` (the grid holds one block, so
// every head's span is that block) the workgroup also finishes the head as
// attn_merge_kernel does for a single partial (o times 1 / l) and writes the
// attention output and its int8 row (qo) itself, so neither the
// qkv_post nor the merge launch is needed.
template <int HD>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void attn_decode_kernel(AttnArgs a,
                                                                                                     QkvArgs qa,
                                                                                                     QOut qo,
                                                                                                     int direct) {
    constexpr int KS = HD + 8, PR = HD / 8;
    extern __shared__ __align__(16) float lds[];
    float* sc = lds;                                   // [256]
    uint16_t* kv = (uint16_t*)(lds + ATTN_BLOCK + 4);  // [256][KS]
    __shared__ float mh, lsh;
    __shared__ __align__(16) float rows[4][HD];  // the token's q head, k and v rows (and a spare)
    const int hh = blockIdx.x, kvh = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = a.G, pw = HD + 2, KVD = a.KV * HD;
    int p0, n_seq, first, last;
    attn_pos(a, p0, n_seq);
    attn_span(a.window, p0, n_seq, first, last);
    const int b = first / ATTN_BLOCK + (int)blockIdx.z;
    if (b > last / ATTN_BLOCK) return;
    const int k0 = first > b * ATTN_BLOCK ? first : b * ATTN_BLOCK;
    const int k1 = last < b * ATTN_BLOCK + ATTN_BLOCK - 1 ? last : b * ATTN_BLOCK + ATTN_BLOCK - 1;
    const int nk = k1 + 1 - k0;
    // Pieces per thread: PR (256 rows), in NB batches. Up to head_dim 128 the
    // V rows have an LDS region of their own and are staged with the K rows;
    // at 256 they replace the K rows after the scores.
    constexpr int U = PR < 16 ? PR : 16, NB = PR / U;
    constexpr bool KV2 = HD <= 128;
    uint16_t* vv = KV2 ? kv + ATTN_BLOCK * KS : kv;
    // The token's own key and value rows are this block's when its position
    // is (a position past the context lies in no block).
    const bool own = p0 >= k0 && p0 <= k1;
    if constexpr (KV2) {
        // The q / k / v rows' reads, then the block's K and V rows', all in
        // flight together (one round trip); the K / V rows are stored to LDS
        // before the q / k / v rows are formed, so their registers are free
        // again by then.
        QkvRegs<HD> g;
        decode_qkv_issue<HD>(qa, g, kvh * G + hh, kvh, p0, wave, lane);
        {
            uint4 rk[U], rv[U];
            kv_load<HD, U>(rk, a.kc, k0, nk, KVD, kvh, tid, 0);
            kv_load<HD, U>(rv, a.vc, k0, nk, KVD, kvh, tid, 0);
            kv_store<HD, U>(rk, kv, tid, 0);
            kv_store<HD, U>(rv, vv, tid, 0);
        }
        decode_qkv_finish<HD>(qa, g, &rows[0][0], own, wave, lane);
    } else {
        decode_qkv_rows<HD>(qa, &rows[0][0], kvh * G + hh, kvh, own, p0, wave, lane);
#pragma unroll
        for (int bt = 0; bt < NB; ++bt) {
            uint4 r[U];
            kv_load<HD, U>(r, a.kc, k0, nk, KVD, kvh, tid, bt * U);
            kv_store<HD, U>(r, kv, tid, bt * U);
        }
    }
    if (own) {
        __syncthreads();  // every staged row is stored: the token's rows replace its stale one
        uint16_t* kd = qa.kc + (size_t)p0 * KVD + kvh * HD;  // the same cache as a.kc, writable
        uint16_t* vd = qa.vc + (size_t)p0 * KVD + kvh * HD;
        for (int i = tid; i < HD; i += 256) {
            const uint16_t kb = to_bf16(rows[1][i]), vb = to_bf16(rows[2][i]);
            kv[(p0 - k0) * KS + i] = kb;
            if (KV2) vv[(p0 - k0) * KS + i] = vb;
            if (hh == 0) {
                kd[i] = kb;
                vd[i] = vb;
            }
        }
    }
    __syncthreads();
    if (tid < nk) {
        const float* qg = &rows[0][0];
        const uint16_t* kr = kv + tid * KS;
        float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < PR; ++c) {
            const uint4 k8 = *(const uint4*)(kr + 8 * c);
            const uint32_t kw[4] = {k8.x, k8.y, k8.z, k8.w};
#pragma unroll
            for (int l = 0; l < 8; ++l)
                acc[l] = __fmaf_rn(qg[8 * c + l], bf16f((kw[l >> 1] >> (16 * (l & 1))) & 0xffffu), acc[l]);
        }
        sc[tid] = __fmul_rn(hsum8(acc), a.scale);
    }
    __syncthreads();
    if (wave == 0) {
        float m = -INFINITY;
        for (int j = 4 * lane; j < 4 * lane + 4 && j < nk; ++j)
            if (m < sc[j]) m = sc[j];
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float other = __shfl_xor(m, o, 64);
            const float lo = (lane & o) ? other : m, hi = (lane & o) ? m : other;
            m = lo < hi ? hi : lo;
        }
        if (lane == 0) mh = sc[0] != sc[0] ? sc[0] : m;
    }
    __syncthreads();
    if (tid < nk) sc[tid] = exp_lane(__fsub_rn(sc[tid], mh));
    __syncthreads();
    float* part = a.parts + ((size_t)kvh * a.nblk + blockIdx.z) * G * pw + hh * pw;
    // The weight sum (lanes 0..7 over the keys in order, hsum8, then the
    // tail): before the V chain at head_dim 256, which takes every thread;
    // up to 128 by wave 3 while waves 0-1 run the V chain.
    auto weight_sum = [&]() {
        const int body = nk & ~7;
        float t[ATTN_BLOCK / 8];
        if (lane < 8) {
#pragma unroll
            for (int k = 0; k < ATTN_BLOCK / 8; ++k) t[k] = sc[lane + 8 * k < body ? lane + 8 * k : 0];
        }
        float vs = 0.0f;
        if (lane < 8) {
#pragma unroll
            for (int k = 0; k < ATTN_BLOCK / 8; ++k)
                if (lane + 8 * k < body) vs = __fadd_rn(vs, t[k]);
        }
        float ls = hsum8_lanes(vs);
        if (lane == 0) {
            for (int j = body; j < nk; ++j) ls = __fadd_rn(ls, sc[j]);
            part[HD] = mh;
            part[HD + 1] = ls;
            lsh = ls;
        }
    };
    if (!KV2 && wave == 0) weight_sum();
    if constexpr (!KV2) {
        // The K rows were last read before the barrier after the scores.
#pragma unroll
        for (int bt = 0; bt < NB; ++bt) {
            uint4 r[U];
            kv_load<HD, U>(r, a.vc, k0, nk, KVD, kvh, tid, bt * U);
            kv_store<HD, U>(r, kv, tid, bt * U);
        }
        if (own) {
            __syncthreads();
            for (int i = tid; i < HD; i += 256) kv[(p0 - k0) * KS + i] = to_bf16(rows[2][i]);
        }
        __syncthreads();
    }
    float o = -0.0f;
    if (tid < HD) {
        // Keys in order, 8 per step, the LDS reads of the next four steps in
        // flight: a ring of four named buffers (no copies), each refilled
        // right after its FMAs with the step four on; the reads are
        // unconditional, clamped to the last whole step, and kept ahead of
        // the FMAs by scheduling barriers.
        constexpr int RING = 4;
        const int body = nk & ~7;
        const uint16_t* vc = vv + tid;
        const auto step = [&](int s) { return s + 8 <= body ? s : body - 8; };
        int j = 0;
        if (body) {
            V8 r[RING];
#pragma unroll
            for (int k = 0; k < RING; ++k) r[k].load<KS>(sc, vc, step(8 * k));
            for (; j + 8 * RING <= body; j += 8 * RING) {
#pragma unroll
                for (int k = 0; k < RING; ++k) {
                    __builtin_amdgcn_sched_barrier(0);
                    o = r[k].fma(o);
                    r[k].load<KS>(sc, vc, step(j + 8 * (RING + k)));
                }
            }
#pragma unroll
            for (int k = 0; k < RING - 1; ++k)
                if (j + 8 <= body) {
                    o = r[k].fma(o);
                    j += 8;
                }
        }
        for (; j < nk; ++j) o = __fmaf_rn(sc[j], bf16f(vv[j * KS + tid]), o);
    } else if (KV2 && wave == 3) {
        weight_sum();
    }
    if constexpr (KV2) __syncthreads();  // lsh
    if (tid < HD) {
        if (direct) {
            // attn_merge_kernel with one partial: o * (1 / l).
            const float al = lsh;
            const float inv = al > 0.0f ? __fdiv_rn(1.0f, al) : 0.0f;
            const float v = __fmul_rn(o, inv);
            const int jo = (kvh * G + hh) * HD + tid;
            a.out[jo] = v;
            if (qo.q) q8_value(v, jo, qo);
        } else {
            part[tid] = o;
        }
    }
}

// The partials of token y's heads sharing KV head x merged in block order
// (scalar.rs:521-537, with glibc's expf), then each head's o / l
// (scalar.rs:539-548) into out[t][head * hd ..]; qo.q != NULL (one token):
// the output also quantized into qo (head_dim a multiple of 32, so every
// half-wave of an iteration holds one block).
__global__ __launch_bounds__(1024) void attn_merge_kernel(AttnArgs a, QOut qo) {
    const int t = blockIdx.y, kvh = blockIdx.x, hd = a.hd, G = a.G, pw = hd + 2, hd8 = hd & ~7;
    int p0, n_seq, first, last;
    attn_pos(a, p0, n_seq);
    attn_span(a.window, p0 + t, n_seq, first, last);
    const int nb = last / ATTN_BLOCK - first / ATTN_BLOCK + 1;
    const float* P = a.parts + ((size_t)t * a.KV + kvh) * a.nblk * G * pw;
    for (int idx = threadIdx.x; idx < G * hd; idx += blockDim.x) {
        const int h = idx / hd, i = idx - h * hd;
        float o = P[h * pw + i], am = P[h * pw + hd], al = P[h * pw + hd + 1];
        for (int bi = 1; bi < nb; ++bi) {
            const float* B = P + (size_t)bi * G * pw + h * pw;
            const float bm = B[hd], bl = B[hd + 1];
            const float m = am < bm ? bm : am;
            const float ca = glibc_expf(__fsub_rn(am, m), a.expt), cb = glibc_expf(__fsub_rn(bm, m), a.expt);
            o = i < hd8 ? __fmaf_rn(B[i], cb, __fmul_rn(o, ca)) : __fadd_rn(__fmul_rn(o, ca), __fmul_rn(B[i], cb));
            am = m;
            al = __fadd_rn(__fmul_rn(al, ca), __fmul_rn(bl, cb));
        }
        const float inv = al > 0.0f ? __fdiv_rn(1.0f, al) : 0.0f;
        const float v = __fmul_rn(o, inv);
        a.out[(size_t)t * (a.KV * G * hd) + (size_t)(kvh * G + h) * hd + i] = v;
        if (qo.q) q8_value(v, kvh * G * hd + idx, qo);
    }
}

// gate = gelu(gate) * up (Gemma) or (gate * sigmoid(gate)) * up, gate and up
// the halves of token y's row of gu [n_tok][2F] (scalar.rs:140-150); four
// values per thread (F a multiple of 32); qo.q != NULL (one token): the
// result also quantized into qo.
__device__ __forceinline__ float act1(float g, float u, int gelu) {
    return gelu ? __fmul_rn(gelu_lane(g), u) : __fmul_rn(__fmul_rn(g, sigmoid_lane(g)), u);
}
__global__ __launch_bounds__(256) void act_kernel(float* __restrict__ gu, int F, int gelu, QOut qo) {
    float4* g = (float4*)(gu + (size_t)blockIdx.y * 2 * F);
    const int i = blockIdx.x * blockDim.x + threadIdx.x, F4 = F / 4;
    const bool ok = i < F4;
    float4 o[1] = {{0.0f, 0.0f, 0.0f, 0.0f}};
    if (ok) {
        const float4 gv = g[i], u = g[F4 + i];
        o[0].x = act1(gv.x, u.x, gelu);
        o[0].y = act1(gv.y, u.y, gelu);
        o[0].z = act1(gv.z, u.z, gelu);
        o[0].w = act1(gv.w, u.w, gelu);
        g[i] = o[0];
    }
    if (qo.q) q8_pieces<1>(o, i, 0, F4, qo);
}

// The argmax row as the next token, recorded, and the position advanced.
__global__ void next_token_kernel(const uint64_t* row, int32_t* tok, int* pos, int32_t* out, int* step) {
    const int32_t t = (int32_t)*row;
    *tok = t;
    out[*step] = t;
    *step += 1;
    *pos += 1;
}

}  // namespace

extern "C" {

struct nngl_model {
    nng_config c;
    std::vector<nnh_weight*> w;  // 7 * n_layer + 1, as nng_gemv_fn's ids; lm_head last
    const nnh_weight* embd = nullptr;
    const uint8_t* table = nullptr;  // the embedding table's split layout (device)
    bool fused_qkv = false, fused_gu = false;
    int act = NNH_ACT_F32, n_batch = 0, nblk = 0;
    size_t pos = 0;
    hipStream_t st = nullptr;
    bool own_stream = false;
    float *norms = nullptr, *bias = nullptr, *cs = nullptr, *sn = nullptr;
    uint64_t* expt = nullptr;
    uint16_t *kc = nullptr, *vc = nullptr;
    float *x = nullptr, *normed = nullptr, *r = nullptr, *qkv = nullptr, *attn = nullptr, *gu = nullptr,
          *parts = nullptr, *states = nullptr, *logits = nullptr;
    int32_t* tok = nullptr;
    int32_t* tok_host = nullptr;  // pinned staging of the host forward's token ids
    void* work = nullptr;
    uint64_t* row = nullptr;
    size_t lds_attn = 0, lds_dec = 0;
    int tq = 1;  // tokens per attention tile
    // One-token forwards in NNH_ACT_I8: the int8 inputs of the matmuls
    // written by their producer kernels (n_embd wide: q/k/v, gate/up and
    // lm_head; the attention output; the FFN activation), one row each in
    // the library's layout at these offsets (s, sx).
    uint8_t *qa_e = nullptr, *qa_a = nullptr, *qa_f = nullptr;
    size_t qo_e[2] = {}, qo_a[2] = {}, qo_f[2] = {};
    bool qfuse = true;    // nngl_set_fused_quant
    bool nfuse = true;    // nngl_set_fused_norm
    float* x2 = nullptr;  // the residual stream's second buffer (fused norms)
    bool q_last = false;  // the last forward left the lm_head input in qa_e
    std::string err;
};

const char* nngl_error(nngl_model* m) { return m ? m->err.c_str() : "no model"; }

void nngl_free(nngl_model* m) {
    if (!m) return;
    void* bufs[] = {m->norms, m->bias, m->cs,    m->sn,     m->expt,   m->kc,     m->vc,   m->x,   m->normed,
                    m->r,     m->qkv,  m->attn, m->gu,     m->parts,  m->states, m->logits, m->tok, m->work, m->row,
                    m->qa_e,  m->qa_a, m->qa_f, m->x2};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    if (m->tok_host) (void)hipHostFree(m->tok_host);
    if (m->own_stream && m->st) (void)hipStreamDestroy(m->st);
    delete m;
}

static size_t norm_stride_l(const nng_config& c) { return 4 * (size_t)c.n_embd + 2 * (size_t)c.head_dim; }

#define NNGL_CHECK(expr)                                                   \
    do {                                                                   \
        hipError_t e_ = (expr);                                            \
        if (e_ != hipSuccess) {                                            \
            m->err = std::string(#expr) + ": " + hipGetErrorString(e_);    \
            return 1;                                                      \
        }                                                                  \
    } while (0)

// RoPE tables as gemma3.cpp's rope forms the angles: ratio = pow(base,
// -2 / n_rot) and inv *= ratio in f32, theta = pos * inv (/ ff[i]), then the
// platform's cosf / sinf.
static void rope_table_l(float base, int n_ctx, int hd, const float* ff, float* cs, float* sn) {
    const int half = hd / 2;
    const float ratio = std::pow(base, -2.0f / (float)hd);
    for (int p = 0; p < n_ctx; ++p) {
        float inv = 1.0f;
        for (int i = 0; i < half; ++i) {
            float theta = (float)p * inv;
            if (ff) theta /= ff[i];
            cs[(size_t)p * half + i] = std::cos(theta);
            sn[(size_t)p * half + i] = std::sin(theta);
            inv *= ratio;
        }
    }
}

// weights: 7 * n_layer + 1 handles with nng_gemv_fn's ids (7 l + {q, k, v,
// o, gate, up, down}, the lm_head last); k and v NULL when q is the fused
// [q; k; v] matrix, up NULL when gate is the fused [gate; up] matrix.
// norms: nng_create's layout; biases: per layer [q_dim][kv_dim][kv_dim] or
// NULL; rope_ff: head_dim / 2 RoPE frequency factors or NULL; token_embd:
// the embedding table (may be the lm_head). n_batch: most tokens per
// forward. act: the matmuls' activation mode. stream: a hipStream_t, or
// NULL for a stream of the model's own.
int nngl_create(const nng_config* cfg, const float* norms, const float* biases, const float* rope_ff,
                nnh_weight* const* weights, int n_weights, const nnh_weight* token_embd, int n_batch, int act,
                void* stream, nngl_model** out) {
    nngl_model* m = new nngl_model();
    *out = m;
    m->c = *cfg;
    const nng_config& c = m->c;
    if (n_weights != 7 * c.n_layer + 1 || c.n_layer < 1 || c.n_kv < 1 || c.n_head % c.n_kv != 0 || n_batch < 1 ||
        n_batch > c.n_ctx) {
        m->err = "bad weight count, head grouping or batch";
        return 1;
    }
    const int E = c.n_embd, hd = c.head_dim, H = c.n_head, KV = c.n_kv, G = H / KV, F = c.n_ff;
    if (E % 32 || E > 8192 || hd % 8 || hd > 512 || F % 32 || G > at_nq(hd) || c.n_vocab < 1 || c.arch < NNG_GEMMA3 ||
        c.arch > NNG_QWEN3) {
        m->err = "n_embd and n_ff must be multiples of 32 (n_embd at most 8192), head_dim a multiple of 8 up to "
                 "512, at most 32 query heads per KV head (16 at head_dim 256)";
        return 1;
    }
    const int QD = H * hd, KVD = KV * hd, QKV = QD + 2 * KVD;
    m->w.assign(weights, weights + n_weights);
    m->fused_qkv = !m->w[1] && !m->w[2];
    m->fused_gu = !m->w[5];
    for (int l = 0; l < c.n_layer; ++l) {
        const bool fq = !m->w[7 * l + 1] && !m->w[7 * l + 2], fg = !m->w[7 * l + 5];
        if (fq != m->fused_qkv || fg != m->fused_gu) {
            m->err = "every layer must fuse q / k / v and gate / up alike";
            return 1;
        }
        const int want[7][2] = {{m->fused_qkv ? QKV : QD, E}, {KVD, E}, {KVD, E}, {E, QD},
                                {m->fused_gu ? 2 * F : F, E}, {F, E}, {E, F}};
        for (int k = 0; k < 7; ++k) {
            const nnh_weight* wk = m->w[7 * l + k];
            if (!wk) {
                if ((k == 1 || k == 2) && m->fused_qkv) continue;
                if (k == 5 && m->fused_gu) continue;
                m->err = "missing weight";
                return 1;
            }
            int dt;
            size_t rows, cols;
            if (nnh_weight_info(wk, &dt, &rows, &cols) != NNH_OK || (int)rows != want[k][0] || (int)cols != want[k][1]) {
                m->err = "layer " + std::to_string(l) + " matrix " + std::to_string(k) + ": shape mismatch";
                return 1;
            }
        }
    }
    {
        int dt;
        size_t rows, cols;
        if (nnh_weight_info(m->w.back(), &dt, &rows, &cols) != NNH_OK || (int)rows != c.n_vocab || (int)cols != E) {
            m->err = "lm_head must be n_vocab x n_embd";
            return 1;
        }
        if (!token_embd || nnh_weight_info(token_embd, &dt, &rows, &cols) != NNH_OK || (int)rows != c.n_vocab ||
            (int)cols != E || (dt != NNH_Q8_0 && dt != NNH_Q4S) || (dt == NNH_Q4S) != (c.wtype == 2)) {
            m->err = "the embedding table must be n_vocab x n_embd, Q4 when wtype is 2, else Q8_0";
            return 1;
        }
    }
    m->embd = token_embd;
    m->table = (const uint8_t*)nnh_weight_device_data(token_embd);
    m->act = act;
    m->n_batch = n_batch;
    m->nblk = (c.n_ctx + ATTN_BLOCK - 1) / ATTN_BLOCK;
    if (hd != 32 && hd != 64 && hd != 128 && hd != 256) {
        m->err = "the attention kernels take head_dim 32, 64, 128 or 256";
        return 1;
    }
    m->tq = G >= at_nq(hd) ? 1 : at_nq(hd) / G;
    const size_t nq = (size_t)m->tq * G;
    m->lds_attn = nq * ATTN_BLOCK * 4 + AT_NQ * 4 + (size_t)AT_KC * (hd + 8) * 2;
    if (m->lds_attn > (size_t)LDS_MAX) {
        m->err = "the attention tile exceeds the LDS";
        return 1;
    }
    if (stream) {
        m->st = (hipStream_t)stream;
    } else {
        NNGL_CHECK(hipStreamCreateWithFlags(&m->st, hipStreamNonBlocking));
        m->own_stream = true;
    }
    const size_t nn = norm_stride_l(c) * c.n_layer + E;
    NNGL_CHECK(hipMalloc(&m->norms, nn * 4));
    NNGL_CHECK(hipMemcpy(m->norms, norms, nn * 4, hipMemcpyHostToDevice));
    if (biases) {
        NNGL_CHECK(hipMalloc(&m->bias, (size_t)c.n_layer * QKV * 4));
        NNGL_CHECK(hipMemcpy(m->bias, biases, (size_t)c.n_layer * QKV * 4, hipMemcpyHostToDevice));
    }
    const size_t half = hd / 2, tab = (size_t)c.n_ctx * half;
    std::vector<float> cs(2 * tab), sn(2 * tab);
    rope_table_l(c.rope_base_swa, c.n_ctx, hd, rope_ff, cs.data(), sn.data());
    rope_table_l(c.rope_base, c.n_ctx, hd, rope_ff, cs.data() + tab, sn.data() + tab);
    NNGL_CHECK(hipMalloc(&m->cs, 2 * tab * 4));
    NNGL_CHECK(hipMalloc(&m->sn, 2 * tab * 4));
    NNGL_CHECK(hipMemcpy(m->cs, cs.data(), 2 * tab * 4, hipMemcpyHostToDevice));
    NNGL_CHECK(hipMemcpy(m->sn, sn.data(), 2 * tab * 4, hipMemcpyHostToDevice));
    uint64_t T[32];
    expf_table(T);
    NNGL_CHECK(hipMalloc(&m->expt, sizeof(T)));
    NNGL_CHECK(hipMemcpy(m->expt, T, sizeof(T), hipMemcpyHostToDevice));
    const size_t cache = (size_t)c.n_layer * c.n_ctx * KVD * 2;
    NNGL_CHECK(hipMalloc(&m->kc, cache));
    NNGL_CHECK(hipMalloc(&m->vc, cache));
    NNGL_CHECK(hipMemset(m->kc, 0, cache));
    NNGL_CHECK(hipMemset(m->vc, 0, cache));
    const size_t nb = n_batch;
    NNGL_CHECK(hipMalloc(&m->x, nb * E * 4));
    NNGL_CHECK(hipMalloc(&m->x2, (size_t)E * 4));
    NNGL_CHECK(hipMalloc(&m->normed, nb * E * 4));
    NNGL_CHECK(hipMalloc(&m->r, nb * E * 4));
    NNGL_CHECK(hipMalloc(&m->qkv, nb * QKV * 4));
    NNGL_CHECK(hipMalloc(&m->attn, nb * QD * 4));
    NNGL_CHECK(hipMalloc(&m->gu, nb * 2 * F * 4));
    NNGL_CHECK(hipMalloc(&m->parts, nb * KV * m->nblk * G * (hd + 2) * 4));
    NNGL_CHECK(hipMalloc(&m->states, (size_t)c.n_layer * E * 4));
    NNGL_CHECK(hipMalloc(&m->logits, (size_t)c.n_vocab * 4));
    NNGL_CHECK(hipMalloc(&m->tok, nb * 4));
    NNGL_CHECK(hipHostMalloc(&m->tok_host, nb * 4));
    NNGL_CHECK(hipMalloc(&m->row, 8));
    if (act == NNH_ACT_I8) {
        uint8_t** bufs[3] = {&m->qa_e, &m->qa_a, &m->qa_f};
        size_t* offs[3] = {m->qo_e, m->qo_a, m->qo_f};
        const int cols[3] = {E, QD, F};
        for (int k = 0; k < 3; ++k) {
            size_t bytes = 0;
            if (nnh_act_layout_ex(NNH_ACT_I8, cols[k], 1, &offs[k][0], &offs[k][1], &bytes) != NNH_OK) {
                m->err = std::string("act layout: ") + nnh_last_error();
                return 1;
            }
            NNGL_CHECK(hipMalloc(bufs[k], bytes));
        }
    }
    const size_t wb = nnh_model_argmax_work_bytes(m->w.back()), ab = nnh_argmax_work_bytes(c.n_vocab);
    NNGL_CHECK(hipMalloc(&m->work, wb > ab ? wb : ab));
    const void* ak = hd == 32 ? (const void*)attn_tile_kernel<32>
                     : hd == 64 ? (const void*)attn_tile_kernel<64>
                     : hd == 128 ? (const void*)attn_tile_kernel<128> : (const void*)attn_tile_kernel<256>;
    NNGL_CHECK(hipFuncSetAttribute(ak, hipFuncAttributeMaxDynamicSharedMemorySize, (int)m->lds_attn));
    m->lds_dec = (size_t)(ATTN_BLOCK + 4) * 4 + (size_t)(hd <= 128 ? 2 : 1) * ATTN_BLOCK * (hd + 8) * 2;
    const void* dk = hd == 32 ? (const void*)attn_decode_kernel<32>
                     : hd == 64 ? (const void*)attn_decode_kernel<64>
                     : hd == 128 ? (const void*)attn_decode_kernel<128>
                                 : (const void*)attn_decode_kernel<256>;
    NNGL_CHECK(hipFuncSetAttribute(dk, hipFuncAttributeMaxDynamicSharedMemorySize, (int)m->lds_dec));
    // The weights' layouts and the stream's scratch for this mode and batch
    // (and for one token), so no forward allocates and a forward can be
    // captured into a graph.
    for (nnh_weight* wk : m->w)
        if (wk && (nnh_stream_reserve(wk, act, nb, m->st) != NNH_OK ||
                   (nb > 1 && nnh_stream_reserve(wk, act, 1, m->st) != NNH_OK))) {
            m->err = std::string("weight layouts: ") + nnh_last_error();
            return 1;
        }
    return 0;
}

static int gemv(nngl_model* m, const nnh_weight* w, const float* x, size_t xs, float* y, size_t ys, size_t n) {
    if (nnh_gemv_batch_dev(w, x, xs, y, ys, n, m->act, m->st) != NNH_OK) {
        m->err = std::string("gemv: ") + nnh_last_error();
        return 1;
    }
    return 0;
}

// The matmul of a one-token forward: on the int8 row `qa` (written by the
// producer kernel) when not NULL, else on the f32 row x.
static int gemv_q(nngl_model* m, const nnh_weight* w, const uint8_t* qa, const float* x, size_t xs, float* y,
                  size_t ys, size_t n) {
    if (!qa) return gemv(m, w, x, xs, y, ys, n);
    if (nnh_gemv_act_dev(w, NNH_ACT_I8, qa, 1, y, ys, m->st) != NNH_OK) {
        m->err = std::string("gemv: ") + nnh_last_error();
        return 1;
    }
    return 0;
}

static QOut qout(uint8_t* base, const size_t* off) {
    return base ? QOut{(int8_t*)base, (uint16_t*)(base + off[0]), (double*)(base + off[1])}
                : QOut{nullptr, nullptr, nullptr};
}

// The forward of n_tok tokens (device ids at tokens_dev) at positions pos0
// .. pos0 + n_tok - 1 (forward.rs:848-965): every layer, the final hidden
// states in the model's x (after the output norm), the K/V rows appended,
// the last token's state after each layer kept. Asynchronous on the model's
// stream; allocates nothing, so it can be captured into a HIP graph. The
// caller keeps positions in order (earlier positions' K/V written first).
// posp (device, or NULL): the first position read by the kernels at run
// time, so one captured step replays at successive positions; the attention
// grid then covers the whole context and the blocks past the span exit.
static int forward_impl(nngl_model* m, const int32_t* tokens_dev, size_t n_tok, size_t pos0, const int* posp) {
    const nng_config& c = m->c;
    if (n_tok == 0 || n_tok > (size_t)m->n_batch || (!posp && pos0 + n_tok > (size_t)c.n_ctx)) {
        m->err = "n_tok out of range or context full";
        return 1;
    }
    const int E = c.n_embd, hd = c.head_dim, H = c.n_head, KV = c.n_kv, G = H / KV, F = c.n_ff;
    const int QD = H * hd, KVD = KV * hd, QKV = QD + 2 * KVD, n = (int)n_tok;
    const bool gemma = c.arch == NNG_GEMMA3, qk_norm = gemma || c.arch == NNG_QWEN3;
    const size_t ns = norm_stride_l(c), half = hd / 2, tab = (size_t)c.n_ctx * half;
    const float embd_scale = gemma ? std::sqrt((float)E) : 1.0f;
    hipStream_t st = m->st;
    // One token in NNH_ACT_I8: the producers quantize the matmul inputs.
    const bool fq = m->qfuse && m->act == NNH_ACT_I8 && n == 1 && m->qa_e;
    uint8_t *qe = fq ? m->qa_e : nullptr, *qt = fq ? m->qa_a : nullptr, *qf = fq ? m->qa_f : nullptr;
    const QOut oe = qout(qe, m->qo_e), oa = qout(qt, m->qo_a), of = qout(qf, m->qo_f);
    m->q_last = false;
    // One token with the fused matrices (Llama / Qwen: no post-norms), in
    // NNH_ACT_F32 or with the producers quantizing in NNH_ACT_I8: each
    // residual add and RMSNorm (and in NNH_ACT_I8 the quantizer) runs in the
    // prologue of the q / k / v or gate / up matmul
    // (nnh_gemv_rmsnorm_act_dev), which writes the new residual stream to
    // the other of two buffers; the last layer's final norm stays a kernel
    // of its own.
    const bool fn = m->nfuse && n == 1 && (m->act == NNH_ACT_F32 || fq) && !gemma && m->fused_qkv && m->fused_gu;
    float *xc = m->x, *xo = m->x2;  // the residual stream and the other buffer
    embed_kernel<<<n, 256, 0, st>>>(tokens_dev, m->table, c.wtype, c.n_vocab, E, embd_scale, m->x);
    if (!fn) launch_resid_norm(m->x, nullptr, nullptr, m->norms, m->normed, nullptr, n, E, c.rms_eps, oe, st);
    NNGL_CHECK(hipGetLastError());
    // One merged output per thread: G * head_dim threads (a multiple of 32)
    // up to 1024, else 1024 threads looping.
    const int merge_threads = G * hd <= 1024 ? G * hd : 1024;
    const int n_seq = posp ? c.n_ctx : (int)(pos0 + n_tok);
    const int nblk = (n_seq - 1) / ATTN_BLOCK + 1;
    for (int li = 0; li < c.n_layer; ++li) {
        const float* nr = m->norms + ns * li;
        const float *q_norm = nr + E, *k_norm = nr + E + hd, *post_attn = nr + E + 2 * hd,
                    *ffn_norm = nr + 2 * E + 2 * hd, *post_ffw = nr + 3 * E + 2 * hd;
        const bool sliding = c.swa_period > 0 && (li + 1) % c.swa_period != 0;  // load.rs:1156-1160
        nnh_weight* const* W = m->w.data() + 7 * li;
        if (fn) {
            // Layer 0 normalises the embedding row; a later layer first adds
            // the previous layer's FFN output and records that state.
            const int rc =
                li == 0 ? nnh_gemv_rmsnorm_act_dev(W[0], m->act, xc, nullptr, nr, c.rms_eps, nullptr, nullptr,
                                                   m->normed, m->qkv, st)
                        : nnh_gemv_rmsnorm_act_dev(W[0], m->act, xc, m->r, nr, c.rms_eps, xo,
                                                   m->states + (size_t)(li - 1) * E, m->normed, m->qkv, st);
            if (rc != NNH_OK) {
                m->err = std::string("gemv rmsnorm: ") + nnh_last_error();
                return 1;
            }
            if (li > 0) std::swap(xc, xo);
        } else if (m->fused_qkv) {
            if (gemv_q(m, W[0], qe, m->normed, E, m->qkv, QKV, n_tok)) return 1;
        } else if (gemv_q(m, W[0], qe, m->normed, E, m->qkv, QKV, n_tok) ||
                   gemv_q(m, W[1], qe, m->normed, E, m->qkv + QD, QKV, n_tok) ||
                   gemv_q(m, W[2], qe, m->normed, E, m->qkv + QD + KVD, QKV, n_tok)) {
            return 1;
        }
        uint16_t* kcl = m->kc + (size_t)li * c.n_ctx * KVD;
        uint16_t* vcl = m->vc + (size_t)li * c.n_ctx * KVD;
        QkvArgs qa{m->qkv,
                   m->bias ? m->bias + (size_t)li * QKV : nullptr,
                   qk_norm ? q_norm : nullptr,
                   qk_norm ? k_norm : nullptr,
                   m->cs + (sliding ? 0 : tab),
                   m->sn + (sliding ? 0 : tab),
                   kcl,
                   vcl,
                   posp,
                   H,
                   KV,
                   hd,
                   QKV,
                   (int)pos0,
                   c.rope_mode,
                   c.n_ctx,
                   c.rms_eps};
        // One token: the attention kernel does qkv_post's work itself and,
        // when the grid is one block, the merge too.
        if (n != 1) qkv_post_kernel<<<dim3(n, H + 2 * KV), 64, (size_t)hd * 4, st>>>(qa);
        AttnArgs aa{m->qkv, kcl, vcl, m->parts, m->attn, m->expt, posp, KV, G, hd, QKV, m->nblk, (int)pos0,
                    n_seq, sliding ? c.window : 0, n, m->tq, c.n_ctx, c.attn_scale};
        const dim3 ag((n + m->tq - 1) / m->tq, KV, nblk);
        const bool direct = n == 1 && nblk == 1;
        if (n == 1) {
            const dim3 dg(G, KV, nblk);
            const int dr = direct ? 1 : 0;
            if (hd == 32)
                attn_decode_kernel<32><<<dg, 256, m->lds_dec, st>>>(aa, qa, oa, dr);
            else if (hd == 64)
                attn_decode_kernel<64><<<dg, 256, m->lds_dec, st>>>(aa, qa, oa, dr);
            else if (hd == 128)
                attn_decode_kernel<128><<<dg, 256, m->lds_dec, st>>>(aa, qa, oa, dr);
            else
                attn_decode_kernel<256><<<dg, 256, m->lds_dec, st>>>(aa, qa, oa, dr);
        } else if (hd == 32)
            attn_tile_kernel<32><<<ag, 256, m->lds_attn, st>>>(aa);
        else if (hd == 64)
            attn_tile_kernel<64><<<ag, 256, m->lds_attn, st>>>(aa);
        else if (hd == 128)
            attn_tile_kernel<128><<<ag, 256, m->lds_attn, st>>>(aa);
        else
            attn_tile_kernel<256><<<ag, 256, m->lds_attn, st>>>(aa);
        if (!direct) attn_merge_kernel<<<dim3(KV, n), merge_threads, 0, st>>>(aa, oa);
        NNGL_CHECK(hipGetLastError());
        if (gemv_q(m, W[3], qt, m->attn, QD, m->r, E, n_tok)) return 1;
        if (fn) {
            if (nnh_gemv_rmsnorm_act_dev(W[4], m->act, xc, m->r, ffn_norm, c.rms_eps, xo, nullptr, m->normed, m->gu,
                                         st) != NNH_OK) {
                m->err = std::string("gemv rmsnorm: ") + nnh_last_error();
                return 1;
            }
            std::swap(xc, xo);
        } else {
            launch_resid_norm(m->x, m->r, gemma ? post_attn : nullptr, ffn_norm, m->normed, nullptr, n, E, c.rms_eps,
                              oe, st);
            if (m->fused_gu) {
                if (gemv_q(m, W[4], qe, m->normed, E, m->gu, 2 * F, n_tok)) return 1;
            } else if (gemv_q(m, W[4], qe, m->normed, E, m->gu, 2 * F, n_tok) ||
                       gemv_q(m, W[5], qe, m->normed, E, m->gu + F, 2 * F, n_tok)) {
                return 1;
            }
        }
        act_kernel<<<dim3((F + 1023) / 1024, n), 256, 0, st>>>(m->gu, F, gemma ? 1 : 0, of);
        NNGL_CHECK(hipGetLastError());
        if (gemv_q(m, W[6], qf, m->gu, 2 * F, m->r, E, n_tok)) return 1;
        const bool last = li + 1 == c.n_layer;
        const float* next = last ? m->norms + ns * c.n_layer : m->norms + ns * (li + 1);
        // Fused: the next layer's q / k / v matmul runs this norm.
        if (!fn || last)
            launch_resid_norm(xc, m->r, gemma ? post_ffw : nullptr, next, last ? m->x : m->normed,
                              m->states + (size_t)li * E, n, E, c.rms_eps, oe, st);
        NNGL_CHECK(hipGetLastError());
    }
    m->q_last = fq;
    return 0;
}

int nngl_forward_dev(nngl_model* m, const int32_t* tokens_dev, size_t n_tok, size_t pos0) {
    return forward_impl(m, tokens_dev, n_tok, pos0, nullptr);
}

// One decode step for replay from a HIP graph: the token at tok_dev (device)
// at the position *pos_dev (device), read when the kernels run. A position
// at or past the context writes nothing and reads no key past it; the caller
// bounds its replays.
int nngl_decode_step_dev(nngl_model* m, const int32_t* tok_dev, const int* pos_dev) {
    return forward_impl(m, tok_dev, 1, 0, pos_dev);
}

// The greedy token after a decode step, on the device: model_argmax of the
// step's hidden state (forward.rs:989-1011) into *tok_dev, out[*step_dev]
// = that token, then *step_dev and *pos_dev advanced. Asynchronous, allocates
// nothing (capturable with the step).
int nngl_greedy_next_dev(nngl_model* m, int32_t* tok_dev, int* pos_dev, int32_t* out, int* step_dev) {
    int rc;
    if (m->act == NNH_ACT_F32) {
        rc = nnh_model_argmax_dev(m->w.back(), m->x, m->logits, m->work, m->row, m->st);
    } else {
        rc = m->q_last ? nnh_gemv_act_dev(m->w.back(), NNH_ACT_I8, m->qa_e, 1, m->logits, m->c.n_vocab, m->st)
                       : nnh_gemv_batch_dev(m->w.back(), m->x, m->c.n_embd, m->logits, m->c.n_vocab, 1, m->act, m->st);
        if (rc == NNH_OK) rc = nnh_argmax_dev(m->logits, m->c.n_vocab, m->work, m->row, m->st);
    }
    if (rc != NNH_OK) {
        m->err = std::string("argmax: ") + nnh_last_error();
        return 1;
    }
    next_token_kernel<<<1, 1, 0, m->st>>>(m->row, tok_dev, pos_dev, out, step_dev);
    NNGL_CHECK(hipGetLastError());
    return 0;
}

// nngl_forward_dev for host token ids at the model's position, which it
// then advances (the ids are checked against the vocabulary first).
int nngl_forward(nngl_model* m, const int32_t* tokens, size_t n_tok) {
    if (n_tok == 0 || n_tok > (size_t)m->n_batch || m->pos + n_tok > (size_t)m->c.n_ctx) {
        m->err = "n_tok out of range or context full";
        return 1;
    }
    for (size_t i = 0; i < n_tok; ++i)
        if (tokens[i] < 0 || tokens[i] >= m->c.n_vocab) {
            m->err = "token outside the vocabulary";
            return 1;
        }
    // The staging buffer is rewritten only once the stream's earlier copies are done.
    NNGL_CHECK(hipStreamSynchronize(m->st));
    memcpy(m->tok_host, tokens, n_tok * 4);
    NNGL_CHECK(hipMemcpyAsync(m->tok, m->tok_host, n_tok * 4, hipMemcpyHostToDevice, m->st));
    if (nngl_forward_dev(m, m->tok, n_tok, m->pos)) return 1;
    m->pos += n_tok;
    return 0;
}

// The greedy token after the last forward of n_tok tokens: model_argmax of
// its last hidden state (forward.rs:989-1011); synchronous.
int nngl_argmax_last(nngl_model* m, size_t n_tok, int32_t* out) {
    if (n_tok == 0 || n_tok > (size_t)m->n_batch) {
        m->err = "n_tok out of range";
        return 1;
    }
    const float* h = m->x + (n_tok - 1) * m->c.n_embd;
    int rc;
    if (m->act == NNH_ACT_F32) {
        rc = nnh_model_argmax_dev(m->w.back(), h, m->logits, m->work, m->row, m->st);
    } else {
        rc = nnh_gemv_batch_dev(m->w.back(), h, m->c.n_embd, m->logits, m->c.n_vocab, 1, m->act, m->st);
        if (rc == NNH_OK) rc = nnh_argmax_dev(m->logits, m->c.n_vocab, m->work, m->row, m->st);
    }
    if (rc != NNH_OK) {
        m->err = std::string("argmax: ") + nnh_last_error();
        return 1;
    }
    uint64_t r = 0;
    NNGL_CHECK(hipMemcpyAsync(&r, m->row, 8, hipMemcpyDeviceToHost, m->st));
    NNGL_CHECK(hipStreamSynchronize(m->st));
    *out = (int32_t)r;
    return 0;
}

// The lm_head row of the last token of a forward of n_tok tokens into
// logits (device, n_vocab floats): model_logits for that token, in the
// model's mode; asynchronous, allocates nothing.
int nngl_logits_last_dev(nngl_model* m, size_t n_tok, float* logits) {
    if (n_tok == 0 || n_tok > (size_t)m->n_batch) {
        m->err = "n_tok out of range";
        return 1;
    }
    return gemv(m, m->w.back(), m->x + (n_tok - 1) * m->c.n_embd, m->c.n_embd, logits, m->c.n_vocab, 1);
}

// Copies out (synchronous; any pointer may be NULL): the final hidden
// states of the last forward (n_tok x n_embd), the last token's state after
// each layer (n_layer x n_embd), the K/V caches (n_layer x n_ctx x kv_dim
// BF16 each).
int nngl_read(nngl_model* m, size_t n_tok, float* hidden, float* states, uint16_t* kcache, uint16_t* vcache) {
    const nng_config& c = m->c;
    if (n_tok > (size_t)m->n_batch) {
        m->err = "n_tok out of range";
        return 1;
    }
    const size_t cache = (size_t)c.n_layer * c.n_ctx * c.n_kv * c.head_dim * 2;
    if (hidden) NNGL_CHECK(hipMemcpyAsync(hidden, m->x, n_tok * c.n_embd * 4, hipMemcpyDeviceToHost, m->st));
    if (states)
        NNGL_CHECK(hipMemcpyAsync(states, m->states, (size_t)c.n_layer * c.n_embd * 4, hipMemcpyDeviceToHost, m->st));
    if (kcache) NNGL_CHECK(hipMemcpyAsync(kcache, m->kc, cache, hipMemcpyDeviceToHost, m->st));
    if (vcache) NNGL_CHECK(hipMemcpyAsync(vcache, m->vc, cache, hipMemcpyDeviceToHost, m->st));
    NNGL_CHECK(hipStreamSynchronize(m->st));
    return 0;
}

size_t nngl_pos(nngl_model* m) { return m->pos; }

// on != 0 (the default): one-token forwards in NNH_ACT_I8 have the kernels
// that produce each matmul's input write it quantized (the same bits as
// the library's quantizer on the f32 row, one launch fewer per matmul);
// 0: every matmul quantizes its f32 input itself.
int nngl_set_fused_quant(nngl_model* m, int on) {
    m->qfuse = on != 0;
    return 0;
}

// on != 0 (the default): one-token forwards with fused q / k / v and
// gate / up matrices, in NNH_ACT_F32 or in NNH_ACT_I8 with the producers
// quantizing (nngl_set_fused_quant), run each residual add and RMSNorm
// inside the next matmul's prologue (nnh_gemv_rmsnorm_act_dev: the same
// bits, one launch fewer per norm); 0: the norm kernel, then the matmul.
int nngl_set_fused_norm(nngl_model* m, int on) {
    m->nfuse = on != 0;
    return 0;
}

// Start the sequence again at position `pos` (0: a new sequence; the
// cache rows past it are overwritten as the forwards reach them).
int nngl_set_pos(nngl_model* m, size_t pos) {
    if (pos > (size_t)m->c.n_ctx) {
        m->err = "position past the context";
        return 1;
    }
    m->pos = pos;
    return 0;
}

}  // extern "C"
