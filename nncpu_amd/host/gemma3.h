// Shared declarations of the model harness (gemma3.cpp: the CPU forward
// with pluggable matmuls; gemma3_gpu.hip: the device-resident Gemma-3
// decode step; layers_gpu.hip: the layer kernels of the device forward).
#pragma once
#include <cstddef>
#include <cstdint>

extern "C" {

// The hyperparameters of a model (model/load.rs:431-595).
struct nng_config {
    int n_layer, n_embd, n_head, n_kv, head_dim, n_ff, n_vocab, n_ctx;
    float rms_eps, rope_base, rope_base_swa, attn_scale;
    int window, swa_period;
    int wtype;  // the matrices' format (the embedding table's too): 2 = Q4, else Q8_0
    // NNG_GEMMA3: embedding rows times sqrt(n_embd), per-head q / k RMSNorm,
    // post-attention and post-FFW RMSNorm, GELU(gate) * up. NNG_LLAMA,
    // NNG_QWEN2, NNG_QWEN3: none of those, SiLU(gate) * up; Qwen2 adds the
    // q / k / v projection biases (nng_set_biases), Qwen3 the per-head q / k
    // RMSNorm. (load.rs:538-566, forward.rs:255-290, 742-809.)
    int arch;
    int rope_mode;  // NNG_ROPE_NEOX (lane i with i + n_rot/2) or NNG_ROPE_NORM (2i with 2i + 1)
};
enum { NNG_GEMMA3 = 0, NNG_LLAMA = 1, NNG_QWEN2 = 2, NNG_QWEN3 = 3 };
enum { NNG_ROPE_NEOX = 0, NNG_ROPE_NORM = 1 };

struct nng_model;
int nng_state(nng_model* m, const uint16_t** kcache, const uint16_t** vcache, size_t* pos, const uint64_t** hashes,
              size_t* n_hashes);
}
