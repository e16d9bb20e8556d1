// Shared declarations of the Gemma-3 decode harness (gemma3.cpp: the CPU
// forward with pluggable matmuls; gemma3_gpu.hip: the device-resident decode
// step).
#pragma once
#include <cstddef>
#include <cstdint>

extern "C" {

// The hyperparameters of a Gemma-3 model (model/load.rs:431-595).
struct nng_config {
    int n_layer, n_embd, n_head, n_kv, head_dim, n_ff, n_vocab, n_ctx;
    float rms_eps, rope_base, rope_base_swa, attn_scale;
    int window, swa_period;
    int wtype;  // the matrices' format (the embedding table's too): 2 = Q4, else Q8_0
};

struct nng_model;
int nng_state(nng_model* m, const uint16_t** kcache, const uint16_t** vcache, size_t* pos, const uint64_t** hashes,
              size_t* n_hashes);
}
