// A Gemma-3 / Llama / Qwen2 / Qwen3 forward pass on the CPU whose every weight
// matmul goes through a pluggable gemv (the reference's `gemv_batch` /
// `model_gemv` dispatch):
// the decode and prefill caller of the quantized matmul, restated from
// crates/nncpu/src/model/forward.rs:197-439 (attention), 719-841 (layer),
// 848-965 (model_forward), 989-1011 (argmax), with the scalar non-matmul
// kernels of crates/nncpu/src/kernels/scalar.rs (norms, GELU, softmax
// pieces of attention) and kernels/mod.rs:687-737 (RoPE).
//
// With the matmul on the GPU (nnh_gemv_batch, bit-exact f32 mode) and the
// rest unchanged, a decode run must give the tokens and the per-layer
// hidden states of the same run with nncpu's CPU gemv: that is the check
// this harness exists for. Built with -ffp-contract=off: std::fma exactly
// where the reference fuses.

#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "gemma3.h"
#include "nncpu_hip.h"

namespace {

// ---- nncpu's scalar kernels (kernels/scalar.rs) ------------------------------------

inline float bf16f(uint16_t v) {
    uint32_t u = (uint32_t)v << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
inline uint16_t to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
inline float hsum8(const float* v) { return ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7])); }

// scalar.rs:19-84: exp(x) as x = n ln2 + r, a degree-5 polynomial for
// exp(r), 2^n in the exponent field (llmcpu's constants).
inline float round_even(float v) {
    volatile float t = v + 12582912.0f;
    return t - 12582912.0f;
}
float exp_lane(float x) {
    const float EXP_LO = -87.336544f, EXP_HI = 88.722839f;
    const float LOG2E = 1.44269504088896340736f, LN2_HI = 0.693359375f, LN2_LO = -2.12194440e-4f;
    const float P[6] = {1.9875691500e-4f, 1.3981999507e-3f, 8.3334519073e-3f,
                        4.1665795894e-2f, 1.6666665459e-1f, 5.0000001201e-1f};
    x = x > EXP_LO ? x : EXP_LO;
    x = x < EXP_HI ? x : EXP_HI;
    float fx = round_even(x * LOG2E);
    float r = std::fma(-fx, LN2_HI, x);
    r = std::fma(-fx, LN2_LO, r);
    float y = std::fma(P[0], r, P[1]);
    y = std::fma(y, r, P[2]);
    y = std::fma(y, r, P[3]);
    y = std::fma(y, r, P[4]);
    y = std::fma(y, r, P[5]);
    y = std::fma(y, r * r, r);
    y = y + 1.0f;
    uint32_t e = (uint32_t)((int32_t)fx + 127) << 23;
    float p2;
    std::memcpy(&p2, &e, 4);
    return y * p2;
}

// scalar.rs:86-103: GELU, tanh form with a Pade [7/6] tanh.
float gelu_lane(float v) {
    const float GELU_C = 0.79788456080286535f, GELU_A = 0.044715f;
    float v3 = (v * v) * v;
    float u = GELU_C * std::fma(GELU_A, v3, v);
    float u2 = u * u, u4 = u2 * u2, u6 = u4 * u2;
    float num = u * (u6 + std::fma(378.0f, u4, std::fma(17325.0f, u2, 135135.0f)));
    float den = std::fma(28.0f, u6, std::fma(3150.0f, u4, std::fma(62370.0f, u2, 135135.0f)));
    float t = std::fabs(u) >= 5.0f ? std::copysign(1.0f, u) : num / den;
    return (0.5f * v) * (1.0f + t);
}

// scalar.rs:104-106: 1 / (1 + exp(0 - g)), a true divide.
float sigmoid_lane(float g) { return 1.0f / (1.0f + exp_lane(0.0f - g)); }

// scalar.rs:146-150: SiLU(gate) * up, in place in gate.
void swiglu(float* gate, const float* up, size_t n) {
    for (size_t i = 0; i < n; ++i) gate[i] = (gate[i] * sigmoid_lane(gate[i])) * up[i];
}

// scalar.rs:232-250: sum of squares, FMA lanes over whole 8-chunks, tail in f64.
double sum_sq(const float* x, size_t n) {
    size_t body = n & ~(size_t)7;
    double s = 0.0;
    if (n >= 8) {
        float acc[8] = {};
        for (size_t i = 0; i < body; i += 8)
            for (int l = 0; l < 8; ++l) acc[l] = std::fma(x[i + l], x[i + l], acc[l]);
        s = (double)hsum8(acc);
    }
    for (size_t i = body; i < n; ++i) s += (double)x[i] * (double)x[i];
    return s;
}

// scalar.rs:270-292: RMSNorm x gamma per group of dim (y may alias x).
void rmsnorm_gamma_multi(float* y, const float* x, size_t total, size_t dim, const float* gamma, float eps) {
    const float inv_dim = 1.0f / (float)dim;
    for (size_t g = 0; g + dim <= total; g += dim) {
        float scale = (float)(1.0 / std::sqrt(sum_sq(x + g, dim) * (double)inv_dim + (double)eps));
        for (size_t i = 0; i < dim; ++i) y[g + i] = (x[g + i] * scale) * gamma[i];
    }
}

// kernels/mod.rs:687-737: RoPE over the first n_rot lanes of each head,
// pairing lane i with i + n_rot/2 (NeoX) or lane 2i with 2i + 1 (Norm); the
// angles pos * base^(-2i/n_rot) (the ratio accumulated in f32), divided by
// the frequency factors ff when given; lanes past n_rot pass through.
void rope(float* x, size_t n_heads, size_t head_dim, size_t n_rot, float pos, float freq_base, int mode,
          const float* ff) {
    if (n_rot == 0) return;
    size_t half = n_rot / 2;
    std::vector<float> cs(half), sn(half);
    float ratio = std::pow(freq_base, -2.0f / (float)n_rot);
    float inv = 1.0f;
    for (size_t i = 0; i < half; ++i) {
        float theta = pos * inv;
        if (ff) theta /= ff[i];
        cs[i] = std::cos(theta);
        sn[i] = std::sin(theta);
        inv *= ratio;
    }
    const size_t stride = mode == NNG_ROPE_NORM ? 2 : 1, partner = mode == NNG_ROPE_NORM ? 1 : half;
    for (size_t h = 0; h < n_heads; ++h) {
        float* xh = x + h * head_dim;
        for (size_t i = 0; i < half; ++i) {
            const size_t p = i * stride;
            float a = xh[p], b = xh[p + partner];
            xh[p] = cs[i] * a - sn[i] * b;
            xh[p + partner] = sn[i] * a + cs[i] * b;
        }
    }
}

constexpr size_t ATTN_BLOCK = 256;  // model/mod.rs:84-87

// scalar.rs:444-519: one block of keys (BF16 K/V rows kv_stride apart) for
// n_heads query heads (q_stride apart) -> partials of hd + 2 floats.
void attn_block(const float* q, size_t q_stride, const uint16_t* kr, const uint16_t* vr, size_t kv_stride,
                size_t n_keys, size_t hd, size_t n_heads, float scale, float* scores, float* part) {
    const size_t pw = hd + 2, hd8 = hd & ~(size_t)7;
    for (size_t t = 0; t < n_keys; ++t) {
        const uint16_t* krow = kr + t * kv_stride;
        for (size_t h = 0; h < n_heads; ++h) {
            const float* qh = q + h * q_stride;
            float acc[8] = {};
            for (size_t i = 0; i < hd8; i += 8)
                for (int l = 0; l < 8; ++l) acc[l] = std::fma(qh[i + l], bf16f(krow[i + l]), acc[l]);
            float s = hsum8(acc);
            for (size_t i = hd8; i < hd; ++i) s = s + qh[i] * bf16f(krow[i]);
            scores[h * n_keys + t] = s * scale;
        }
    }
    const size_t body = n_keys & ~(size_t)7;
    for (size_t h = 0; h < n_heads; ++h) {
        float* s = scores + h * n_keys;
        float m = s[0];
        for (size_t i = 1; i < n_keys; ++i)
            if (m < s[i]) m = s[i];
        float vsum[8] = {};
        for (size_t i = 0; i < body; i += 8)
            for (int l = 0; l < 8; ++l) {
                s[i + l] = exp_lane(s[i + l] - m);
                vsum[l] += s[i + l];
            }
        float lsum = hsum8(vsum);
        for (size_t i = body; i < n_keys; ++i) {
            s[i] = exp_lane(s[i] - m);
            lsum += s[i];
        }
        part[h * pw + hd] = m;
        part[h * pw + hd + 1] = lsum;
    }
    for (size_t t = 0; t < n_keys; ++t) {
        const uint16_t* vrow = vr + t * kv_stride;
        for (size_t h = 0; h < n_heads; ++h) {
            const float w = scores[h * n_keys + t];
            float* o = part + h * pw;
            if (t == 0) {
                for (size_t i = 0; i < hd; ++i) o[i] = w * bf16f(vrow[i]);
            } else {
                for (size_t i = 0; i < hd8; ++i) o[i] = std::fma(w, bf16f(vrow[i]), o[i]);
                for (size_t i = hd8; i < hd; ++i) o[i] += w * bf16f(vrow[i]);
            }
        }
    }
}

// scalar.rs:521-537
void attn_merge(float* acc, const float* part, size_t hd, size_t n_heads) {
    const size_t pw = hd + 2, hd8 = hd & ~(size_t)7;
    for (size_t h = 0; h < n_heads; ++h) {
        float* a = acc + h * pw;
        const float* b = part + h * pw;
        float m = a[hd] < b[hd] ? b[hd] : a[hd];
        float ca = std::exp(a[hd] - m), cb = std::exp(b[hd] - m);
        for (size_t i = 0; i < hd8; ++i) a[i] = std::fma(b[i], cb, a[i] * ca);
        for (size_t i = hd8; i < hd; ++i) a[i] = a[i] * ca + b[i] * cb;
        a[hd] = m;
        a[hd + 1] = a[hd + 1] * ca + b[hd + 1] * cb;
    }
}

// scalar.rs:539-548
void attn_finish(float* out, size_t out_stride, const float* acc, size_t hd, size_t n_heads) {
    const size_t pw = hd + 2;
    for (size_t h = 0; h < n_heads; ++h) {
        float l = acc[h * pw + hd + 1];
        float inv = l > 0.0f ? 1.0f / l : 0.0f;
        for (size_t i = 0; i < hd; ++i) out[h * out_stride + i] = acc[h * pw + i] * inv;
    }
}

// model/embed.rs:14-30, the causal branch.
void attn_span(size_t window, size_t pos, size_t n_seq, size_t* first, size_t* last) {
    size_t end = n_seq ? n_seq - 1 : 0;
    *first = (window > 0 && pos + 1 > window) ? pos + 1 - window : 0;
    *last = pos < end ? pos : end;
}

}  // namespace

extern "C" {


// y (n_tok vectors, y_stride apart) = matrix `id` x (x_stride apart), the
// gemv_batch contract; returns 0 on success. id = 7*layer + {0 q, 1 k, 2 v,
// 3 o, 4 gate, 5 up, 6 down}; 7*n_layer is the (tied) lm_head.
typedef int (*nng_gemv_fn)(void* ctx, int id, const float* x, size_t x_stride, float* y, size_t y_stride,
                           size_t n_tok);
// The lm_head argmax of one hidden state (model_argmax); may be NULL, then
// the harness takes the logits through the gemv and an argmax of its own.
typedef int (*nng_argmax_fn)(void* ctx, const float* x, size_t* row);

struct nng_model {
    nng_config c;
    std::vector<float> norms;          // per layer: attn, q, k, post_attn, ffn, post_ffw; then output
    std::vector<float> bias;           // per layer: q, k, v projection biases (Qwen2), or empty
    std::vector<float> rope_ff;        // RoPE frequency factors (head_dim / 2), or empty
    std::vector<uint8_t> token_embd;   // Q8_0 or Q4 split layout [n_vocab x n_embd] (the embedding table)
    nng_gemv_fn gemv;
    nng_argmax_fn argmax;
    void* ctx;
    // state
    std::vector<uint16_t> kcache, vcache;  // [n_layer][n_ctx][kv_dim] BF16
    size_t cur_pos = 0;
    std::vector<float> x, normed, q, k, v, attn, gate, up, scores, part, acc, logits;
    std::vector<uint64_t> layer_hash;  // FNV-1a of each layer's output residual, last token of each forward
    std::string err;
};

static size_t norm_stride(const nng_config& c) { return 4 * (size_t)c.n_embd + 2 * (size_t)c.head_dim; }

// norms: per layer [attn n_embd][q_norm hd][k_norm hd][post_attn n_embd][ffn n_embd][post_ffw n_embd],
// then output_norm [n_embd]. token_embd: the split layout of the embedding / lm_head table (Q4 when
// cfg->wtype is 2, else Q8_0).
nng_model* nng_create(const nng_config* cfg, const float* norms, const void* token_embd, nng_gemv_fn gemv,
                      nng_argmax_fn argmax, void* ctx) {
    nng_model* m = new nng_model();
    m->c = *cfg;
    const nng_config& c = m->c;
    size_t nn = norm_stride(c) * c.n_layer + c.n_embd;
    m->norms.assign(norms, norms + nn);
    size_t te = (size_t)c.n_vocab * c.n_embd;
    const size_t tbytes = c.wtype == 2 ? te / 2 + te / 8 : te + te / 16;
    m->token_embd.assign((const uint8_t*)token_embd, (const uint8_t*)token_embd + tbytes);
    m->gemv = gemv;
    m->argmax = argmax;
    m->ctx = ctx;
    size_t kv_dim = (size_t)c.n_kv * c.head_dim;
    m->kcache.assign((size_t)c.n_layer * c.n_ctx * kv_dim, 0);
    m->vcache.assign((size_t)c.n_layer * c.n_ctx * kv_dim, 0);
    return m;
}

void nng_free(nng_model* m) { delete m; }

// The q / k / v projection biases (Qwen2, forward.rs:255-272): per layer
// [q_dim][kv_dim][kv_dim] floats, added to the projections before the
// norms and RoPE.
void nng_set_biases(nng_model* m, const float* b) {
    const nng_config& c = m->c;
    const size_t per = (size_t)(c.n_head + 2 * c.n_kv) * c.head_dim;
    m->bias.assign(b, b + per * c.n_layer);
}

// RoPE frequency factors (head_dim / 2 floats; Llama 3's long-context
// scaling, load.rs:760-769), or NULL for none.
void nng_set_rope_freqs(nng_model* m, const float* ff) {
    if (ff)
        m->rope_ff.assign(ff, ff + m->c.head_dim / 2);
    else
        m->rope_ff.clear();
}
const char* nng_error(nng_model* m) { return m->err.c_str(); }

static uint64_t fnv(const float* v, size_t n) {
    uint64_t h = 1469598103934665603ull;
    const uint8_t* p = (const uint8_t*)v;
    for (size_t i = 0; i < 4 * n; ++i) h = (h ^ p[i]) * 1099511628211ull;
    return h;
}

// The per-layer hash the forward records (FNV-1a of the residual's bytes),
// for hidden states recorded elsewhere: count states of n floats each.
void nng_fnv_many(const float* v, size_t n, size_t count, uint64_t* out) {
    for (size_t i = 0; i < count; ++i) out[i] = fnv(v + i * n, n);
}

// Row `tok` of a split-layout embedding table times `scale` into y[0..E)
// (model/mod.rs:447-460): Q8_0 f32(q) * (s * scale) (kernels/mod.rs:917-930);
// Q4 (wtype 2) (s * scale) * q + bias * scale, unfused, byte k of a block
// holding elements k (low nibble) and k + 16 (kernels/mod.rs:934-954).
static void embed_row(int wtype, const uint8_t* table, size_t n_vocab, size_t E, size_t tok, float scale, float* y) {
    const size_t te = n_vocab * E, nbe = E / 32;
    if (wtype == 2) {
        const uint8_t* tq = table + tok * (E / 2);
        const uint16_t* ts = (const uint16_t*)(table + te / 2) + tok * nbe;
        const uint16_t* tb = (const uint16_t*)(table + te / 2 + te / 16) + tok * nbe;
        for (size_t b = 0; b < nbe; ++b) {
            const float s = bf16f(ts[b]) * scale, bias = bf16f(tb[b]) * scale;
            for (int k = 0; k < 16; ++k) {
                const uint8_t q = tq[16 * b + k];
                y[32 * b + k] = s * (float)(q & 15) + bias;
                y[32 * b + k + 16] = s * (float)(q >> 4) + bias;
            }
        }
    } else {
        const int8_t* tq = (const int8_t*)table + tok * E;
        const uint16_t* ts = (const uint16_t*)(table + te) + tok * nbe;
        for (size_t b = 0; b < nbe; ++b) {
            const float vs = bf16f(ts[b]) * scale;
            for (int i = 0; i < 32; ++i) y[32 * b + i] = (float)tq[32 * b + i] * vs;
        }
    }
}

// model_forward (forward.rs:848-965) for n_tok tokens at cur_pos.
int nng_forward(nng_model* m, const int32_t* tokens, size_t n_tok) {
    const nng_config& c = m->c;
    const size_t E = c.n_embd, hd = c.head_dim, H = c.n_head, KV = c.n_kv, F = c.n_ff;
    const size_t q_dim = H * hd, kv_dim = KV * hd, pos0 = m->cur_pos;
    if (n_tok == 0 || pos0 + n_tok > (size_t)c.n_ctx) {
        m->err = "context full";
        return 1;
    }
    m->x.assign(n_tok * E, 0.0f);
    m->normed.assign(n_tok * E, 0.0f);
    m->q.assign(n_tok * q_dim, 0.0f);
    m->k.assign(n_tok * kv_dim, 0.0f);
    m->v.assign(n_tok * kv_dim, 0.0f);
    m->attn.assign(n_tok * q_dim, 0.0f);
    m->gate.assign(n_tok * F, 0.0f);
    m->up.assign(n_tok * F, 0.0f);
    const size_t group = H / KV, pw = hd + 2;
    m->scores.assign(group * ATTN_BLOCK, 0.0f);
    m->part.assign(group * pw, 0.0f);
    m->acc.assign(group * pw, 0.0f);

    // Embedding rows times sqrt(n_embd) for Gemma, else 1 (load.rs:565-566).
    const bool gemma = c.arch == NNG_GEMMA3, qk_norm = gemma || c.arch == NNG_QWEN3;
    const float embd_scale = gemma ? std::sqrt((float)E) : 1.0f;
    const float* ff = m->rope_ff.empty() ? nullptr : m->rope_ff.data();
    for (size_t t = 0; t < n_tok; ++t) {
        if (tokens[t] < 0 || tokens[t] >= c.n_vocab) {
            m->err = "token outside the vocabulary";
            return 1;
        }
        embed_row(c.wtype, m->token_embd.data(), (size_t)c.n_vocab, E, (size_t)tokens[t], embd_scale,
                  m->x.data() + t * E);
    }

    const size_t ns = norm_stride(c);
    for (int li = 0; li < c.n_layer; ++li) {
        const float* nr = m->norms.data() + ns * li;
        const float *attn_norm = nr, *q_norm = nr + E, *k_norm = nr + E + hd, *post_attn = nr + E + 2 * hd,
                    *ffn_norm = nr + 2 * E + 2 * hd, *post_ffw = nr + 3 * E + 2 * hd;
        const bool sliding = c.swa_period > 0 && (li + 1) % c.swa_period != 0;  // load.rs:1156-1160
        const int id = 7 * li;
        // attention block
        rmsnorm_gamma_multi(m->normed.data(), m->x.data(), n_tok * E, E, attn_norm, c.rms_eps);
        if (m->gemv(m->ctx, id + 0, m->normed.data(), E, m->q.data(), q_dim, n_tok) ||
            m->gemv(m->ctx, id + 1, m->normed.data(), E, m->k.data(), kv_dim, n_tok) ||
            m->gemv(m->ctx, id + 2, m->normed.data(), E, m->v.data(), kv_dim, n_tok)) {
            m->err = "gemv failed";
            return 1;
        }
        if (!m->bias.empty()) {  // forward.rs:255-272
            const float* bl = m->bias.data() + (q_dim + 2 * kv_dim) * li;
            for (size_t t = 0; t < n_tok; ++t) {
                for (size_t i = 0; i < q_dim; ++i) m->q[t * q_dim + i] += bl[i];
                for (size_t i = 0; i < kv_dim; ++i) m->k[t * kv_dim + i] += bl[q_dim + i];
                for (size_t i = 0; i < kv_dim; ++i) m->v[t * kv_dim + i] += bl[q_dim + kv_dim + i];
            }
        }
        if (qk_norm) {  // forward.rs:274-290: Gemma, Qwen3
            rmsnorm_gamma_multi(m->q.data(), m->q.data(), n_tok * q_dim, hd, q_norm, c.rms_eps);
            rmsnorm_gamma_multi(m->k.data(), m->k.data(), n_tok * kv_dim, hd, k_norm, c.rms_eps);
        }
        const float freq = sliding ? c.rope_base_swa : c.rope_base;
        for (size_t t = 0; t < n_tok; ++t) {
            float rpos = (float)(pos0 + t);
            rope(m->q.data() + t * q_dim, H, hd, hd, rpos, freq, c.rope_mode, ff);
            rope(m->k.data() + t * kv_dim, KV, hd, hd, rpos, freq, c.rope_mode, ff);
        }
        // Append K/V as BF16 (forward.rs:326-351); rows = n_ctx, no ring wrap below n_ctx.
        uint16_t* kc = m->kcache.data() + (size_t)li * c.n_ctx * kv_dim;
        uint16_t* vc = m->vcache.data() + (size_t)li * c.n_ctx * kv_dim;
        for (size_t t = 0; t < n_tok; ++t)
            for (size_t i = 0; i < kv_dim; ++i) {
                kc[(pos0 + t) * kv_dim + i] = to_bf16(m->k[t * kv_dim + i]);
                vc[(pos0 + t) * kv_dim + i] = to_bf16(m->v[t * kv_dim + i]);
            }
        const size_t n_seq = pos0 + n_tok, window = sliding ? (size_t)c.window : 0;
        for (size_t t = 0; t < n_tok; ++t) {
            size_t first, last;
            attn_span(window, pos0 + t, n_seq, &first, &last);
            for (size_t kvh = 0; kvh < KV; ++kvh) {
                const float* qg = m->q.data() + t * q_dim + kvh * group * hd;
                for (size_t b = first / ATTN_BLOCK; b <= last / ATTN_BLOCK; ++b) {
                    size_t k0 = first > b * ATTN_BLOCK ? first : b * ATTN_BLOCK;
                    size_t k1 = last < b * ATTN_BLOCK + ATTN_BLOCK - 1 ? last : b * ATTN_BLOCK + ATTN_BLOCK - 1;
                    size_t off = k0 * kv_dim + kvh * hd;
                    float* dst = b == first / ATTN_BLOCK ? m->acc.data() : m->part.data();
                    attn_block(qg, hd, kc + off, vc + off, kv_dim, k1 + 1 - k0, hd, group, c.attn_scale,
                               m->scores.data(), dst);
                    if (b != first / ATTN_BLOCK) attn_merge(m->acc.data(), m->part.data(), hd, group);
                }
                attn_finish(m->attn.data() + t * q_dim + kvh * group * hd, hd, m->acc.data(), hd, group);
            }
        }
        if (m->gemv(m->ctx, id + 3, m->attn.data(), q_dim, m->normed.data(), E, n_tok)) {
            m->err = "gemv failed";
            return 1;
        }
        if (gemma) rmsnorm_gamma_multi(m->normed.data(), m->normed.data(), n_tok * E, E, post_attn, c.rms_eps);
        for (size_t i = 0; i < n_tok * E; ++i) m->x[i] += m->normed[i];
        // MLP block: gelu(gate) * up (Gemma) or silu(gate) * up, then down
        // (forward.rs:755-803).
        rmsnorm_gamma_multi(m->normed.data(), m->x.data(), n_tok * E, E, ffn_norm, c.rms_eps);
        if (m->gemv(m->ctx, id + 4, m->normed.data(), E, m->gate.data(), F, n_tok) ||
            m->gemv(m->ctx, id + 5, m->normed.data(), E, m->up.data(), F, n_tok)) {
            m->err = "gemv failed";
            return 1;
        }
        if (gemma)
            for (size_t i = 0; i < n_tok * F; ++i) m->gate[i] = gelu_lane(m->gate[i]) * m->up[i];
        else
            swiglu(m->gate.data(), m->up.data(), n_tok * F);
        if (m->gemv(m->ctx, id + 6, m->gate.data(), F, m->normed.data(), E, n_tok)) {
            m->err = "gemv failed";
            return 1;
        }
        if (gemma) rmsnorm_gamma_multi(m->normed.data(), m->normed.data(), n_tok * E, E, post_ffw, c.rms_eps);
        for (size_t i = 0; i < n_tok * E; ++i) m->x[i] += m->normed[i];
        m->layer_hash.push_back(fnv(m->x.data() + (n_tok - 1) * E, E));
    }
    rmsnorm_gamma_multi(m->x.data(), m->x.data(), n_tok * E, E, m->norms.data() + ns * c.n_layer, c.rms_eps);
    m->cur_pos = pos0 + n_tok;
    return 0;
}

// The decode state after the forwards so far: KV caches ([n_layer][n_ctx]
// [kv_dim] BF16), the next position, and the per-layer hashes recorded.
int nng_state(nng_model* m, const uint16_t** kcache, const uint16_t** vcache, size_t* pos, const uint64_t** hashes,
              size_t* n_hashes) {
    if (kcache) *kcache = m->kcache.data();
    if (vcache) *vcache = m->vcache.data();
    if (pos) *pos = m->cur_pos;
    if (hashes) *hashes = m->layer_hash.data();
    if (n_hashes) *n_hashes = m->layer_hash.size();
    return 0;
}

// Greedy choice from the last token's final hidden state (forward.rs:989-1011).
int nng_argmax_last(nng_model* m, size_t n_tok, int32_t* out) {
    const size_t E = m->c.n_embd;
    const float* hidden = m->x.data() + (n_tok - 1) * E;
    if (m->argmax) {
        size_t row = 0;
        if (m->argmax(m->ctx, hidden, &row)) {
            m->err = "argmax failed";
            return 1;
        }
        *out = (int32_t)row;
        return 0;
    }
    m->logits.assign(m->c.n_vocab, 0.0f);
    if (m->gemv(m->ctx, 7 * m->c.n_layer, hidden, E, m->logits.data(), m->c.n_vocab, 1)) {
        m->err = "gemv failed";
        return 1;
    }
    size_t best = 0;
    for (size_t i = 1; i < (size_t)m->c.n_vocab; ++i)
        if (m->logits[i] > m->logits[best]) best = i;
    *out = (int32_t)best;
    return 0;
}

// A prompt in batches of `batch` tokens (session/engine.rs:362-380,
// PREFILL_BATCH = 16), then n_gen greedy tokens (engine.rs:598-695).
// out_tokens gets the n_gen tokens; hashes (if not NULL) the per-layer
// hashes of every forward call, n_layer per call, in order.
// t_prefill / t_decode (if not NULL) get the seconds spent before and after
// the first generated token.
int nng_generate(nng_model* m, const int32_t* prompt, size_t n_prompt, size_t batch, size_t n_gen,
                 int32_t* out_tokens, uint64_t* hashes, size_t* n_hashes, double* t_prefill, double* t_decode) {
    auto t0 = std::chrono::steady_clock::now();
    m->cur_pos = 0;
    m->layer_hash.clear();
    size_t last_n = 0;
    for (size_t p = 0; p < n_prompt; p += batch) {
        size_t n = n_prompt - p < batch ? n_prompt - p : batch;
        if (nng_forward(m, prompt + p, n)) return 1;
        last_n = n;
    }
    int32_t tok;
    if (nng_argmax_last(m, last_n, &tok)) return 1;
    auto t1 = std::chrono::steady_clock::now();
    for (size_t g = 0; g < n_gen; ++g) {
        out_tokens[g] = tok;
        if (g + 1 == n_gen) break;
        if (nng_forward(m, &tok, 1)) return 1;
        if (nng_argmax_last(m, 1, &tok)) return 1;
    }
    auto t2 = std::chrono::steady_clock::now();
    if (t_prefill) *t_prefill = std::chrono::duration<double>(t1 - t0).count();
    if (t_decode) *t_decode = std::chrono::duration<double>(t2 - t1).count();
    if (hashes) std::memcpy(hashes, m->layer_hash.data(), m->layer_hash.size() * 8);
    if (n_hashes) *n_hashes = m->layer_hash.size();
    return 0;
}

// ---- the GPU matmul backend: the library's C-ABI --------------------------------------

struct nng_gpu_ctx {
    nnh_weight** w;  // 7 * n_layer + 1 weights, lm_head last
    int n;
    int act;
};

int nng_gpu_gemv(void* ctx, int id, const float* x, size_t x_stride, float* y, size_t y_stride, size_t n_tok) {
    nng_gpu_ctx* g = (nng_gpu_ctx*)ctx;
    if (id < 0 || id >= g->n) return 1;
    return nnh_gemv_batch(g->w[id], x, x_stride, y, y_stride, n_tok, g->act) != NNH_OK;
}

int nng_gpu_argmax(void* ctx, const float* x, size_t* row) {
    nng_gpu_ctx* g = (nng_gpu_ctx*)ctx;
    return nnh_model_argmax(g->w[g->n - 1], x, row, g->act) != NNH_OK;
}

// ---- the forward's non-matmul ops, one by one ------------------------------------------
// The functions the forward above calls (and the device decode step repeats
// operation for operation), exported so the reference's own op tests can be
// run against them (crates/nncpu/src/kernels/tests.rs:105-147, 242-293,
// 938-992, 1133-1217, 1263).

// std::exp of floats, as attn_merge takes it (the platform libm's expf).
void nng_op_embed_row(int wtype, const void* table, size_t n_vocab, size_t n_embd, size_t token, float scale,
                      float* y) {
    embed_row(wtype, (const uint8_t*)table, n_vocab, n_embd, token, scale, y);
}

void nng_op_libm_expf(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = std::exp(x[i]);
}

void nng_op_exp(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = exp_lane(x[i]);
}

void nng_op_gelu(float* x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = gelu_lane(x[i]);
}

// gelu(gate) * up, in place in gate (the forward's MLP step).
void nng_op_gelu_mul(float* gate, const float* up, size_t n) {
    for (size_t i = 0; i < n; ++i) gate[i] = gelu_lane(gate[i]) * up[i];
}

void nng_op_rmsnorm_gamma(float* y, const float* x, size_t total, size_t dim, const float* gamma, float eps) {
    rmsnorm_gamma_multi(y, x, total, dim, gamma, eps);
}

void nng_op_rope_neox(float* x, size_t n_heads, size_t head_dim, size_t n_rot, float pos, float freq_base) {
    rope(x, n_heads, head_dim, n_rot, pos, freq_base, NNG_ROPE_NEOX, nullptr);
}

// mode: NNG_ROPE_NEOX or NNG_ROPE_NORM; ff: n_rot / 2 frequency factors or NULL.
void nng_op_rope(float* x, size_t n_heads, size_t head_dim, size_t n_rot, float pos, float freq_base, int mode,
                 const float* ff) {
    rope(x, n_heads, head_dim, n_rot, pos, freq_base, mode, ff);
}

// SiLU(gate) * up, in place in gate (the Llama / Qwen MLP step).
void nng_op_swiglu(float* gate, const float* up, size_t n) { swiglu(gate, up, n); }

// n_keys <= 256 (one block); scores holds n_heads * n_keys floats, part
// n_heads * (hd + 2).
void nng_op_attn_block(const float* q, size_t q_stride, const uint16_t* kr, const uint16_t* vr, size_t kv_stride,
                       size_t n_keys, size_t hd, size_t n_heads, float scale, float* scores, float* part) {
    attn_block(q, q_stride, kr, vr, kv_stride, n_keys, hd, n_heads, scale, scores, part);
}

void nng_op_attn_merge(float* acc, const float* part, size_t hd, size_t n_heads) {
    attn_merge(acc, part, hd, n_heads);
}

void nng_op_attn_finish(float* out, size_t out_stride, const float* acc, size_t hd, size_t n_heads) {
    attn_finish(out, out_stride, acc, hd, n_heads);
}

}  // extern "C"
