// The Gemma-3 decode step resident on the GPU: the forward of gemma3.cpp
// (crates/nncpu/src/model/forward.rs:197-439, 719-965 with the scalar.rs
// non-matmul kernels) for one token, with every operation in the same order
// and rounding as that CPU restatement, so a decode gives the same tokens and
// the same per-layer hidden states bit for bit. The weight matmuls are the
// library's bit-exact f32 path (nnh_gemv_batch_dev), the lm_head argmax is
// nnh_argmax_dev, the token and the position live in device memory, and one
// step is captured once in a HIP graph and replayed per generated token: no
// host round trip inside the decode loop.
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

#include "gemma3.h"
#include "nncpu_hip.h"

namespace {

constexpr int ATTN_BLOCK = 256;  // model/mod.rs:84-87

__device__ __forceinline__ float bf16f(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }
__device__ __forceinline__ uint16_t to_bf16(float f) {
    const uint32_t u = __float_as_uint(f);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float hsum8(const float* v) {
    return __fadd_rn(__fadd_rn(__fadd_rn(v[0], v[4]), __fadd_rn(v[1], v[5])),
                     __fadd_rn(__fadd_rn(v[2], v[6]), __fadd_rn(v[3], v[7])));
}

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

// RMSNorm x gamma of one group of `dim` values by the whole workgroup
// (scalar.rs:232-292, gemma3.cpp sum_sq / rmsnorm_gamma_multi): eight FMA
// lanes over whole chunks of 8, hsum8, the tail in f64, scale
// (float)(1 / sqrt(ss * inv_dim + eps)) in f64. y may alias x.
__device__ void rmsnorm_wg(const float* x, const float* gamma, float* y, int dim, float eps) {
    __shared__ float lanes[8];
    __shared__ float scale_s;
    const int body = dim & ~7;
    if (threadIdx.x < 8) {
        float a = 0.0f;
        for (int i = 0; i < body; i += 8) a = __fmaf_rn(x[i + threadIdx.x], x[i + threadIdx.x], a);
        lanes[threadIdx.x] = a;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double s = dim >= 8 ? (double)hsum8(lanes) : 0.0;
        for (int i = body; i < dim; ++i) s = __dadd_rn(s, __dmul_rn((double)x[i], (double)x[i]));
        const float inv_dim = __fdiv_rn(1.0f, (float)dim);
        scale_s = (float)__ddiv_rn(1.0, __dsqrt_rn(__dadd_rn(__dmul_rn(s, (double)inv_dim), (double)eps)));
    }
    __syncthreads();
    const float scale = scale_s;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) y[i] = __fmul_rn(__fmul_rn(x[i], scale), gamma[i]);
    __syncthreads();
}

// ---- the step's kernels -----------------------------------------------------------------

// Embedding row times sqrt(n_embd) (kernels/mod.rs:917-929): the Q8_0 row of
// the tied token_embd, f32(q) * (bf16(s) * scale).
__global__ void embed_kernel(const uint64_t* tok, const int8_t* tq, const uint16_t* ts, int E, float embd_scale,
                             float* x) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= E) return;
    const size_t t = (size_t)*tok;
    const float vs = __fmul_rn(bf16f(ts[t * (E / 32) + i / 32]), embd_scale);
    x[i] = __fmul_rn((float)tq[t * E + i], vs);
}

__global__ void rmsnorm_kernel(const float* x, const float* gamma, float* y, int dim, float eps) {
    rmsnorm_wg(x, gamma, y, dim, eps);
}

// Per head: q / k RMSNorm, NeoX RoPE at the current position, then the K/V
// append to the BF16 caches (forward.rs:326-351). Workgroups 0..H-1 take the
// query heads, H..H+KV-1 the key heads.
__global__ void qk_kernel(float* q, float* k, const float* v, const float* q_norm, const float* k_norm,
                          const float* cos_t, const float* sin_t, const int* pos_p, uint16_t* kc, uint16_t* vc,
                          int H, int KV, int hd, float eps) {
    const int pos = *pos_p;
    const int head = blockIdx.x;
    const bool is_q = head < H;
    float* x = is_q ? q + head * hd : k + (head - H) * hd;
    rmsnorm_wg(x, is_q ? q_norm : k_norm, x, hd, eps);
    const int half = hd / 2;
    const float* cs = cos_t + (size_t)pos * half;
    const float* sn = sin_t + (size_t)pos * half;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const float a = x[i], b = x[i + half];
        x[i] = __fsub_rn(__fmul_rn(cs[i], a), __fmul_rn(sn[i], b));
        x[i + half] = __fadd_rn(__fmul_rn(sn[i], a), __fmul_rn(cs[i], b));
    }
    if (!is_q) {
        __syncthreads();
        const int kvh = head - H, kv_dim = KV * hd;
        for (int i = threadIdx.x; i < hd; i += blockDim.x) {
            kc[(size_t)pos * kv_dim + kvh * hd + i] = to_bf16(x[i]);
            vc[(size_t)pos * kv_dim + kvh * hd + i] = to_bf16(v[kvh * hd + i]);
        }
    }
}

// One query head over its key span, in one key block (attn_block,
// attn_finish: scalar.rs:444-548): scores by 8-lane FMA dots and hsum8,
// times the attention scale; the first-maximum; exp_lane; the 8-lane sum of
// the weights over whole chunks, hsum8, then the tail in order; the V sum
// as one FMA chain per output element over the keys in order; / sum.
__global__ __launch_bounds__(256) void attn_kernel(const float* q, const uint16_t* kc, const uint16_t* vc,
                                                   const int* pos_p, int group, int KV, int hd, int window,
                                                   float scale, float* out) {
    __shared__ float sc[ATTN_BLOCK];
    __shared__ float vsum[8];
    __shared__ float m_s, inv_s;
    const int pos = *pos_p, h = blockIdx.x, kvh = h / group;
    const int first = (window > 0 && pos + 1 > window) ? pos + 1 - window : 0;
    const int n_keys = pos + 1 - first;
    const int kv_dim = KV * hd, hd8 = hd & ~7;
    const float* qh = q + h * hd;
    for (int t = threadIdx.x; t < n_keys; t += blockDim.x) {
        const uint16_t* krow = kc + (size_t)(first + t) * kv_dim + kvh * hd;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int i = 0; i < hd8; i += 8)
#pragma unroll
            for (int l = 0; l < 8; ++l) acc[l] = __fmaf_rn(qh[i + l], bf16f(krow[i + l]), acc[l]);
        float s = hsum8(acc);
        for (int i = hd8; i < hd; ++i) s = __fadd_rn(s, __fmul_rn(qh[i], bf16f(krow[i])));
        sc[t] = __fmul_rn(s, scale);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = sc[0];
        for (int i = 1; i < n_keys; ++i)
            if (m < sc[i]) m = sc[i];
        m_s = m;
    }
    __syncthreads();
    const float m = m_s;
    for (int t = threadIdx.x; t < n_keys; t += blockDim.x) sc[t] = exp_lane(__fsub_rn(sc[t], m));
    __syncthreads();
    const int body = n_keys & ~7;
    if (threadIdx.x < 8) {
        float a = 0.0f;
        for (int i = 0; i < body; i += 8) a = __fadd_rn(a, sc[i + threadIdx.x]);
        vsum[threadIdx.x] = a;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float l = hsum8(vsum);
        for (int i = body; i < n_keys; ++i) l = __fadd_rn(l, sc[i]);
        inv_s = l > 0.0f ? __fdiv_rn(1.0f, l) : 0.0f;
    }
    __syncthreads();
    const float inv = inv_s;
    for (int i = threadIdx.x; i < hd; i += blockDim.x) {
        const uint16_t* vcol = vc + (size_t)first * kv_dim + kvh * hd + i;
        float o = __fmul_rn(sc[0], bf16f(vcol[0]));
        if (i < hd8) {
            for (int t = 1; t < n_keys; ++t) o = __fmaf_rn(sc[t], bf16f(vcol[(size_t)t * kv_dim]), o);
        } else {
            for (int t = 1; t < n_keys; ++t) o = __fadd_rn(o, __fmul_rn(sc[t], bf16f(vcol[(size_t)t * kv_dim])));
        }
        out[h * hd + i] = __fmul_rn(o, inv);
    }
}

// x += RMSNorm(o, post); y = RMSNorm(x, next) (forward.rs:749-803): the
// post-attention / post-FFW norm, the residual, and the next norm. When
// `record` is set, x is also copied there (the per-layer hidden state).
__global__ __launch_bounds__(1024) void residual_kernel(float* o, float* x, const float* post, const float* next,
                                                        float* y, int E, float eps, float* record,
                                                        const int* step_p, int rec_stride) {
    rmsnorm_wg(o, post, o, E, eps);
    for (int i = threadIdx.x; i < E; i += blockDim.x) x[i] = __fadd_rn(x[i], o[i]);
    __syncthreads();
    if (record) {
        float* r = record + (size_t)*step_p * rec_stride;
        for (int i = threadIdx.x; i < E; i += blockDim.x) r[i] = x[i];
    }
    rmsnorm_wg(x, next, y, E, eps);
}

__global__ void gelu_mul_kernel(float* gate, const float* up, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) gate[i] = __fmul_rn(gelu_lane(gate[i]), up[i]);
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

}  // namespace

extern "C" {

struct nngd_model {
    nng_config c;
    std::vector<nnh_weight*> w;  // 7 * n_layer + 1, lm_head (the tied token_embd) last
    float* norms = nullptr;      // device copy, layout of nng_create
    uint16_t *kc = nullptr, *vc = nullptr;
    float *cos_t = nullptr, *sin_t = nullptr;  // [2][n_ctx][hd/2]: sliding (local) base, then global
    float *x = nullptr, *y = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr, *o = nullptr;
    float *gate = nullptr, *up = nullptr, *logits = nullptr, *record = nullptr;
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
    void* bufs[] = {m->norms, m->kc, m->vc, m->cos_t, m->sin_t, m->x, m->y, m->q, m->k, m->v, m->attn, m->o,
                    m->gate, m->up, m->logits, m->record, m->work, m->tok, m->pos, m->step, m->tokens};
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
    m->w.assign(weights, weights + n_weights);
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
    GD_HIP(hipMalloc((void**)&m->x, E * 4));
    GD_HIP(hipMalloc((void**)&m->y, E * 4));
    GD_HIP(hipMalloc((void**)&m->o, E * 4));
    GD_HIP(hipMalloc((void**)&m->q, qd * 4));
    GD_HIP(hipMalloc((void**)&m->k, kvd * 4));
    GD_HIP(hipMalloc((void**)&m->v, kvd * 4));
    GD_HIP(hipMalloc((void**)&m->attn, qd * 4));
    GD_HIP(hipMalloc((void**)&m->gate, (size_t)c.n_ff * 4));
    GD_HIP(hipMalloc((void**)&m->up, (size_t)c.n_ff * 4));
    GD_HIP(hipMalloc((void**)&m->logits, (size_t)c.n_vocab * 4));
    GD_HIP(hipMalloc((void**)&m->record, (size_t)n_gen_max * c.n_layer * E * 4));
    GD_HIP(hipMalloc(&m->work, nnh_argmax_work_bytes((size_t)c.n_vocab)));
    GD_HIP(hipMalloc((void**)&m->tok, 8));
    GD_HIP(hipMalloc((void**)&m->pos, 4));
    GD_HIP(hipMalloc((void**)&m->step, 4));
    GD_HIP(hipMalloc((void**)&m->tokens, (size_t)n_gen_max * 4));
    return 0;
}

// Queue one decode step on m->st (eagerly, or into a graph being captured).
static int queue_step(nngd_model* m) {
    const nng_config& c = m->c;
    const int E = c.n_embd, hd = c.head_dim, H = c.n_head, KV = c.n_kv, F = c.n_ff;
    const size_t ns = norm_stride(c);
    hipStream_t st = m->st;
    const uint8_t* te = (const uint8_t*)nnh_weight_device_data(m->w.back());
    const int8_t* tq = (const int8_t*)te;
    const uint16_t* ts = (const uint16_t*)(te + (size_t)c.n_vocab * E);
    const float eps = c.rms_eps;
    embed_kernel<<<(E + 255) / 256, 256, 0, st>>>(m->tok, tq, ts, E, std::sqrt((float)E), m->x);
    rmsnorm_kernel<<<1, 1024, 0, st>>>(m->x, m->norms, m->y, E, eps);
    for (int li = 0; li < c.n_layer; ++li) {
        const float* nr = m->norms + ns * li;
        const float *q_norm = nr + E, *k_norm = nr + E + hd, *post_attn = nr + E + 2 * hd,
                    *ffn_norm = nr + 2 * E + 2 * hd, *post_ffw = nr + 3 * E + 2 * hd;
        const float* next = li + 1 < c.n_layer ? m->norms + ns * (li + 1) : m->norms + ns * c.n_layer;
        const bool sliding = c.swa_period > 0 && (li + 1) % c.swa_period != 0;  // load.rs:1156-1160
        const size_t half = hd / 2, tab = sliding ? 0 : (size_t)c.n_ctx * half;
        nnh_weight* const* w = m->w.data() + 7 * li;
        const size_t kvd = (size_t)KV * hd, cache = (size_t)li * c.n_ctx * kvd;
        if (nnh_gemv_batch_dev(w[0], m->y, E, m->q, H * hd, 1, NNH_ACT_F32, st) ||
            nnh_gemv_batch_dev(w[1], m->y, E, m->k, kvd, 1, NNH_ACT_F32, st) ||
            nnh_gemv_batch_dev(w[2], m->y, E, m->v, kvd, 1, NNH_ACT_F32, st)) {
            m->err = std::string("gemv: ") + nnh_last_error();
            return 1;
        }
        qk_kernel<<<H + KV, 256, 0, st>>>(m->q, m->k, m->v, q_norm, k_norm, m->cos_t + tab, m->sin_t + tab, m->pos,
                                          m->kc + cache, m->vc + cache, H, KV, hd, eps);
        attn_kernel<<<H, 256, 0, st>>>(m->q, m->kc + cache, m->vc + cache, m->pos, H / KV, KV, hd,
                                       sliding ? c.window : 0, c.attn_scale, m->attn);
        if (nnh_gemv_batch_dev(w[3], m->attn, H * hd, m->o, E, 1, NNH_ACT_F32, st)) {
            m->err = std::string("gemv: ") + nnh_last_error();
            return 1;
        }
        residual_kernel<<<1, 1024, 0, st>>>(m->o, m->x, post_attn, ffn_norm, m->y, E, eps, nullptr, nullptr, 0);
        if (nnh_gemv_batch_dev(w[4], m->y, E, m->gate, F, 1, NNH_ACT_F32, st) ||
            nnh_gemv_batch_dev(w[5], m->y, E, m->up, F, 1, NNH_ACT_F32, st)) {
            m->err = std::string("gemv: ") + nnh_last_error();
            return 1;
        }
        gelu_mul_kernel<<<(F + 255) / 256, 256, 0, st>>>(m->gate, m->up, F);
        if (nnh_gemv_batch_dev(w[6], m->gate, F, m->o, E, 1, NNH_ACT_F32, st)) {
            m->err = std::string("gemv: ") + nnh_last_error();
            return 1;
        }
        residual_kernel<<<1, 1024, 0, st>>>(m->o, m->x, post_ffw, next, m->y, E, eps, m->record + (size_t)li * E,
                                            m->step, c.n_layer * E);
    }
    // y = RMSNorm(x, output_norm): the greedy token is the lm_head argmax of y.
    if (nnh_gemv_batch_dev(m->w.back(), m->y, E, m->logits, c.n_vocab, 1, NNH_ACT_F32, st) ||
        nnh_argmax_dev(m->logits, (size_t)c.n_vocab, m->work, m->tok, st)) {
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
